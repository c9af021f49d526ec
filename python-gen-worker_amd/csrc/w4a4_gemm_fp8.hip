// W4A4 GEMM on gfx950's fp8 MFMA, with the weights prepacked once.
//
// Every int4 product of a K-group is computed exactly by ONE
// v_mfma_scale_f32_32x32x64_f8f6f4 (fp8 e4m3 operands, fp32 accumulate):
//
//  * weights are prepacked (gwa_svdq_pack_weight_int4) into a "rotated
//    sign-magnitude" nibble layout: for a packed dword w,
//        lo = w & 0x87878787,  hi = rotr(w, 4) & 0x87878787
//    are four fp8 bytes each whose value is exactly q_w * 2^-9 (e4m3
//    subnormals: sign bit 7, magnitude in bits 0..2), q_w in [-7, 7];
//  * activations keep the two's-complement int4 contract; XOR 0x8 turns a
//    nibble into u = q_x + 8 in [0, 15], and the byte u is the e4m3 value
//    u * 2^-9 (subnormals and the first normal binade are evenly spaced);
//  * with the E8M0 operand scale 2^6 on the weights, the MFMA returns
//    sum_k q_w (q_x + 8) * 2^-12 = (P + 8 * cw) * 2^-12 exactly, where P is
//    the group's integer dot product and cw = sum_k q_w.
//
// Dequantization, per group g, 32x32 block and element (n, m):
//    acc += (P + 8 cw) 2^-12 * sw'[n] sx[m]          (S = sw' (x) sx: f16 MFMA, exact;
//                                                      one VALU fma per element)
//    acc += sum_{g in stage} (-c'_g[n]) sx_g[m]       (one f16 MFMA per 4 groups)
// with c'_g[n] = cw_g[n] sw'_g[n] 2^-9 prepacked as an f16 hi + lo pair, so
// the offset term 8 cw drops out to about 2^-22 of c'. sw' = sw * 2^-e[n]
// is the weight scale rescaled by a per-row power of two (exact) so that
// both sw' and c' sit well inside the f16 range; the epilogue multiplies by
// 2^12 * 2^e[n] * s2 * second[n], adds la @ up^T (bf16 MFMA), bias, optional
// GELU, and stores four consecutive n per lane.
//
// Tiling: a 512-thread workgroup owns a 128 (n) x 256 (m) tile; its 8 waves
// form a 2 x 4 grid of 64 x 64 wave tiles (2 x 2 blocks of 32 x 32), two
// waves per SIMD so one wave's MFMAs overlap the other's VALU work. A stage
// is 4 K-groups (128 bytes of every packed row, so each load instruction
// covers whole 128-byte lines of 8 rows); LDS is double buffered with the
// activations as int4 and the weights already expanded to fp8 by the loader
// (each weight row holds the even-k bytes of the stage's 8 half-groups, then
// their odd-k bytes). Each group's operands are read from LDS while the
// previous group's MFMAs and dequantization run.
// Tiles are ordered so that each XCD (workgroup id mod 8) works on a compact
// block of the output and its operands stay in that XCD's L2.
#include "gwa_common.h"

namespace {

constexpr int TN = 128, TM = 256;
constexpr int WBN = 2, WBM = 2;
constexpr int WAVES_N = TN / (32 * WBN), WAVES_M = TM / (32 * WBM);
constexpr int NTHREADS = 64 * WAVES_N * WAVES_M;  // 512
constexpr int GS = 4;                              // groups per stage
constexpr int KTB = GS * 32;                       // packed bytes per row per stage (128)
constexpr int XSTR = KTB + 16;                     // LDS row stride, activations (int4)
constexpr int WSTR = 2 * KTB + 16;                 // LDS row stride, weights (fp8)
constexpr int LDS_X = TM * XSTR;                   // 36864
constexpr int LDS_W = TN * WSTR;                   // 34816
constexpr int LDS_SX = TM * GS * 2;                // [TM][GS] f16
constexpr int LDS_SW = TN * GS * 2;                // [TN][GS] f16
constexpr int LDS_CW = TN * 16;                    // [TN][hi0..3, lo0..3] f16
constexpr int OFF_W = LDS_X, OFF_SX = OFF_W + LDS_W, OFF_SW = OFF_SX + LDS_SX, OFF_CW = OFF_SW + LDS_SW;
constexpr int LDS_STAGE = OFF_CW + LDS_CW;         // 76800
constexpr int OFF_EPI = 2 * LDS_STAGE;             // [TN] column multipliers, [TN] bias (fp32)
constexpr int LDS_TOTAL = OFF_EPI + 2 * TN * 4;
static_assert(TM * KTB / 16 == 4 * NTHREADS && TN * KTB / 16 == 2 * NTHREADS, "loader split");
constexpr int kWScaleE8M0 = 127 + 6;               // 2^6 on the weight operand
constexpr float kUnscale = 4096.0f;                // 2^12
constexpr int kXcds = 8;

__device__ __forceinline__ uint32_t rotr4(uint32_t w) { return __builtin_amdgcn_alignbit(w, w, 4); }

// 4 packed weight dwords (32 codes) -> 8 fp8 dwords: the even-k codes, then the odd-k codes
__device__ __forceinline__ v8i wgt_fp8(v4i p) {
  v8i r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = (uint32_t)p[j];
    r[j] = (int)(w & 0x87878787u);
    r[4 + j] = (int)(rotr4(w) & 0x87878787u);
  }
  return r;
}

// 4 activation dwords (32 codes) -> 8 fp8 dwords holding q + 8, same k order
__device__ __forceinline__ v8i act_fp8(v4i p) {
  v8i r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = (uint32_t)p[j];
    r[j] = (int)((w ^ 0x88888888u) & 0x0F0F0F0Fu);
    r[4 + j] = (int)(((w >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu);
  }
  return r;
}

// (P + 8 cw) * 2^-12 + c for one group: A = weight rows, B = activation rows
__device__ __forceinline__ v16f group_mfma_fp8(v8i a, v8i b, v16f c = (v16f){}) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, kWScaleE8M0, 0, 127);
}

// f16 operand with the scale in K slot 0 (lanes 0..31) and zeros elsewhere
__device__ __forceinline__ v4h scale_operand(uint16_t s_bits, int h) {
  const uint32_t lo = h == 0 ? (uint32_t)s_bits : 0u;
  typedef unsigned int v2u __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(v4h, (v2u){lo, 0u});
}

__device__ __forceinline__ uint2 buf_load8(rsrc_t r, uint32_t off) {
  typedef unsigned int v2u __attribute__((ext_vector_type(2)));
  const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return make_uint2(v[0], v[1]);
}

// workgroup id -> (tile_m, tile_n): a contiguous run of tiles per XCD, in an
// order that walks GM tile rows before moving to the next tile column
__device__ __forceinline__ bool tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
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

template <int RB, bool GELU, bool OUT_F16>
__global__ __launch_bounds__(NTHREADS, 1) void w4a4_gemm_fp8_kernel(
    const uint8_t* __restrict__ qa, const uint16_t* __restrict__ sa, const uint8_t* __restrict__ qwp,
    const uint16_t* __restrict__ swp, const uint16_t* __restrict__ wcorr, const float* __restrict__ escale,
    const float* __restrict__ s2p, const float* __restrict__ second, int second_per_channel,
    const uint16_t* __restrict__ la, const uint16_t* __restrict__ up, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x;
  const int tiles_n = (N + TN - 1) / TN, tiles_m = (M + TM - 1) / TM;
  int tm, tn;
  if (!tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn)) return;  // whole workgroup, before any barrier
  const int n0 = tn * TN, m0 = tm * TM;
  const int kbytes = K >> 1, G = K >> 6;
  const int nstages = G / GS;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wn = wave % WAVES_N, wm = wave / WAVES_N;
  const int r32 = lane & 31, h = lane >> 5;

  const rsrc_t wbuf = make_rsrc(qwp, (uint32_t)((int64_t)N * kbytes));
  const rsrc_t xbuf = make_rsrc(qa, (uint32_t)((int64_t)M * kbytes));
  // scale / correction staging is split by wave (buffer descriptors are wave-uniform):
  // waves 0-3 the activation scales, 4-5 the weight scales, 6-7 the correction pairs
  const int srole = wave < 4 ? 0 : (wave < 6 ? 1 : 2);
  const int srow = srole == 0 ? tid : (srole == 1 ? tid - 256 : tid - 384);
  const rsrc_t sbuf = srole == 0 ? make_rsrc(sa, (uint32_t)((int64_t)M * G * 2))
                                 : (srole == 1 ? make_rsrc(swp, (uint32_t)((int64_t)N * G * 2))
                                               : make_rsrc(wcorr, (uint32_t)((int64_t)N * G * 4)));
  const uint32_t soff = srole == 0 ? (uint32_t)((int64_t)(m0 + srow) * G * 2)
                                   : (srole == 1 ? (uint32_t)((int64_t)(n0 + srow) * G * 2)
                                                 : (uint32_t)((int64_t)(n0 + srow) * G * 4));
  const uint32_t sstep = srole == 2 ? 16u : 8u;

  // loader roles: 8 lanes per row, 16 bytes each
  const int lrow = tid >> 3, lc = tid & 7;
  uint32_t xoff[4], woff[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) xoff[j] = (uint32_t)((int64_t)(m0 + lrow + 64 * j) * kbytes + lc * 16);
#pragma unroll
  for (int j = 0; j < 2; ++j) woff[j] = (uint32_t)((int64_t)(n0 + lrow + 64 * j) * kbytes + lc * 16);

  struct Stage {
    v4i x[4], w[2], s;
  };
  auto load = [&](Stage& r, int st) {
    const uint32_t kb = (uint32_t)(st * KTB);
#pragma unroll
    for (int j = 0; j < 4; ++j) r.x[j] = buf_load16(xbuf, xoff[j] + kb);
#pragma unroll
    for (int j = 0; j < 2; ++j) r.w[j] = buf_load16(wbuf, woff[j] + kb);
    if (srole == 2) {
      r.s = buf_load16(sbuf, soff + st * sstep);
    } else {
      const uint2 v = buf_load8(sbuf, soff + st * sstep);
      r.s = (v4i){(int)v.x, (int)v.y, 0, 0};
    }
  };
  auto store = [&](const Stage& r, int buf) {
    uint8_t* base = lds + buf * LDS_STAGE;
#pragma unroll
    for (int j = 0; j < 4; ++j) *(v4i*)(base + (lrow + 64 * j) * XSTR + lc * 16) = r.x[j];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const v8i f = wgt_fp8(r.w[j]);
      uint8_t* d = base + OFF_W + (lrow + 64 * j) * WSTR + lc * 16;
      *(v4i*)(d) = (v4i){f[0], f[1], f[2], f[3]};
      *(v4i*)(d + KTB) = (v4i){f[4], f[5], f[6], f[7]};
    }
    if (srole == 0) {
      *(uint2*)(base + OFF_SX + srow * 8) = make_uint2((uint32_t)r.s[0], (uint32_t)r.s[1]);
    } else if (srole == 1) {
      *(uint2*)(base + OFF_SW + srow * 8) = make_uint2((uint32_t)r.s[0], (uint32_t)r.s[1]);
    } else {
      *(v4i*)(base + OFF_CW + srow * 16) = r.s;
    }
  };

  v16f acc[WBN][WBM];
#pragma unroll
  for (int a = 0; a < WBN; ++a)
#pragma unroll
    for (int b = 0; b < WBM; ++b) acc[a][b] = (v16f){};

  Stage regs;
  load(regs, 0);
  // the tile's per-column epilogue constants, staged once: 2^12 * s2 * 2^e[n] * second[n] and bias[n]
  if (tid < TN) {
    const int n = n0 + tid;
    float mult = 0.0f, bv = 0.0f;
    if (n < N) {
      mult = (s2p ? *s2p : 1.0f) * kUnscale * escale[n];
      if (second) mult *= second[second_per_channel ? n : 0];
      if (bias) bv = bf16_to_f32(bias[n]);
    }
    float* epi = (float*)(lds + OFF_EPI);
    epi[tid] = mult;
    epi[TN + tid] = bv;
  }
  store(regs, 0);
  __syncthreads();

  for (int st = 0; st < nstages; ++st) {
    const int buf = st & 1;
    if (st + 1 < nstages) load(regs, st + 1);
    const uint8_t* base = lds + buf * LDS_STAGE;
    const uint8_t* lx = base;
    const uint8_t* lw = base + OFF_W;
    // the stage's scales: 4 groups per row, one 8-byte read per block
    uint2 sxv[WBM], swv[WBN];
#pragma unroll
    for (int bm = 0; bm < WBM; ++bm) sxv[bm] = *(const uint2*)(base + OFF_SX + (32 * (WBM * wm + bm) + r32) * 8);
#pragma unroll
    for (int bn = 0; bn < WBN; ++bn) swv[bn] = *(const uint2*)(base + OFF_SW + (32 * (WBN * wn + bn) + r32) * 8);
    // operand registers for group gi (cur) and gi + 1 (next)
    v4i xr[2][WBM], wr[2][WBN][2];
    auto fetch = [&](int slot, int gi) {
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm)
        xr[slot][bm] = *(const v4i*)(lx + (32 * (WBM * wm + bm) + r32) * XSTR + gi * 32 + 16 * h);
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn) {
        const uint8_t* wp = lw + (32 * (WBN * wn + bn) + r32) * WSTR + (2 * gi + h) * 16;
        wr[slot][bn][0] = *(const v4i*)(wp);
        wr[slot][bn][1] = *(const v4i*)(wp + KTB);
      }
    };
    fetch(0, 0);
#pragma unroll
    for (int gi = 0; gi < GS; ++gi) {
      const int cur = gi & 1;
      if (gi + 1 < GS) fetch(cur ^ 1, gi + 1);
      v8i bx[WBM];
      v4h bs[WBM];
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm) {
        bx[bm] = act_fp8(xr[cur][bm]);
        const uint32_t sw2 = gi < 2 ? sxv[bm].x : sxv[bm].y;
        bs[bm] = scale_operand((uint16_t)((gi & 1) ? sw2 >> 16 : sw2), h);
      }
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn) {
        const v4i w0 = wr[cur][bn][0], w1 = wr[cur][bn][1];
        const v8i aw = (v8i){w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
        const uint32_t s2w = gi < 2 ? swv[bn].x : swv[bn].y;
        const v4h as = scale_operand((uint16_t)((gi & 1) ? s2w >> 16 : s2w), h);
#pragma unroll
        for (int bm = 0; bm < WBM; ++bm) {
          const v16f p = group_mfma_fp8(aw, bx[bm]);
          const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs[bm], (v16f){}, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[bn][bm][v] = fmaf(p[v], sc[v], acc[bn][bm][v]);
        }
      }
    }
    // offset correction for the stage's 4 groups: K slots 0..3 hold -c' hi, 4..7 hold -c' lo
    {
      v4h cb[WBM];
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm) cb[bm] = __builtin_bit_cast(v4h, sxv[bm]);
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn) {
        const int nrow = 32 * (WBN * wn + bn) + r32;
        const v4h ca = *(const v4h*)(base + OFF_CW + nrow * 16 + 8 * h);
#pragma unroll
        for (int bm = 0; bm < WBM; ++bm)
          acc[bn][bm] = __builtin_amdgcn_mfma_f32_32x32x8f16(ca, cb[bm], acc[bn][bm], 0, 0, 0);
      }
    }
    if (st + 1 < nstages) store(regs, buf ^ 1);
    __syncthreads();
  }

  // ---------------- epilogue ----------------
  // acc = acc * colmul[n]; acc += la @ up^T (the low-rank operands loaded in
  // chunks of up to 2 rank-16 slices, every load of a chunk in flight
  // together); then + bias[n] (+ GELU) and packed stores.
  const float* epi = (const float*)(lds + OFF_EPI);
#pragma unroll
  for (int bn = 0; bn < WBN; ++bn) {
    const int nl = 32 * (WBN * wn + bn);  // block's first column within the tile
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const v4f cm = *(const v4f*)(epi + nl + 8 * qd + 4 * h);
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[bn][bm][4 * qd + e] *= cm[e];
    }
  }
  if (RB > 0) {
    constexpr int RC = RB < 2 ? RB : 2;
    const rsrc_t ubuf = make_rsrc(up, (uint32_t)((int64_t)N * RB * 32));
    const rsrc_t lbuf = make_rsrc(la, (uint32_t)((int64_t)M * RB * 32));
#pragma unroll
    for (int k0 = 0; k0 < RB; k0 += RC) {
      v4i ua[WBN][RC > 0 ? RC : 1], lb[WBM][RC > 0 ? RC : 1];
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn)
#pragma unroll
        for (int kk = 0; kk < RC; ++kk)
          ua[bn][kk] = buf_load16(
              ubuf, (uint32_t)((int64_t)(n0 + 32 * (WBN * wn + bn) + r32) * (RB * 32) + (k0 + kk) * 32 + 16 * h));
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm)
#pragma unroll
        for (int kk = 0; kk < RC; ++kk)
          lb[bm][kk] = buf_load16(
              lbuf, (uint32_t)((int64_t)(m0 + 32 * (WBM * wm + bm) + r32) * (RB * 32) + (k0 + kk) * 32 + 16 * h));
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn)
#pragma unroll
        for (int bm = 0; bm < WBM; ++bm)
#pragma unroll
          for (int kk = 0; kk < RC; ++kk)
            acc[bn][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ua[bn][kk]),
                                                                  __builtin_bit_cast(v8bf, lb[bm][kk]), acc[bn][bm],
                                                                  0, 0, 0);
    }
  }
  const rsrc_t obuf = make_rsrc(out, (uint32_t)((int64_t)M * N * 2));
#pragma unroll
  for (int bn = 0; bn < WBN; ++bn) {
    const int nl = 32 * (WBN * wn + bn);
#pragma unroll
    for (int bm = 0; bm < WBM; ++bm) {
      const int m = m0 + 32 * (WBM * wm + bm) + r32;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int n = n0 + nl + 8 * qd + 4 * h;
        const v4f cb = *(const v4f*)(epi + TN + nl + 8 * qd + 4 * h);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = acc[bn][bm][4 * qd + e] + cb[e];
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
        // branch-free store after the MFMAs: rows >= M / columns >= N fall outside the buffer
        const uint32_t off = (m < M && n < N) ? (uint32_t)(((int64_t)m * N + n) * 2) : kOOB;
        buf_store8(pk, obuf, off);
      }
    }
  }
}

// Exact per-group partial sums through the same fp8 path (debug / parity).
__global__ __launch_bounds__(64) void w4a4_psums_fp8_kernel(const uint8_t* __restrict__ qa,
                                                            const uint8_t* __restrict__ qwp,
                                                            const int16_t* __restrict__ wsum,
                                                            int32_t* __restrict__ out, int M, int N, int K) {
  const int lane = threadIdx.x, r32 = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
  const int kbytes = K >> 1, G = K >> 6;
  const int m = m0 + r32, nr = n0 + r32;
  const rsrc_t obuf = make_rsrc(out, (uint32_t)((int64_t)M * N * G * 4));
  for (int g = 0; g < G; ++g) {
    const v4i a = nr < N ? *(const v4i*)(qwp + (int64_t)nr * kbytes + g * 32 + 16 * h) : (v4i){0, 0, 0, 0};
    const v4i b = m < M ? *(const v4i*)(qa + (int64_t)m * kbytes + g * 32 + 16 * h) : (v4i){0, 0, 0, 0};
    v16f dc;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int n = n0 + 8 * (v >> 2) + 4 * h + (v & 3);
      dc[v] = n < N ? -(float)wsum[(int64_t)n * G + g] * (1.0f / 512.0f) : 0.0f;
    }
    const v16f p = group_mfma_fp8(wgt_fp8(a), act_fp8(b), dc);
    // no branch after the MFMA (a sunk MFMA would run with lanes disabled):
    // out-of-range rows/columns are dropped by the buffer bounds instead
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int n = n0 + 8 * (v >> 2) + 4 * h + (v & 3);
      const uint32_t off = (m < M && n < N) ? (uint32_t)((((int64_t)m * N + n) * G + g) * 4) : kOOB;
      buf_store4((uint32_t)(int32_t)(p[v] * kUnscale), obuf, off);
    }
  }
}

// Prepack, one 64-thread block per weight row n:
//  * logical two's-complement codes -> rotated sign-magnitude layout, plus the
//    per-group code sums cw (int16) and a count of -8 codes (which this
//    layout cannot hold);
//  * e[n] = floor(log2(max_g sw[n][g])) - 14, sw' = sw * 2^-e[n] (f16, exact
//    unless a group's scale is 2^25 or more below the row's largest) and
//    escale[n] = 2^e[n];
//  * -c'_g = -cw_g * sw'_g * 2^-9 (exact in fp32) as f16 hi + lo, stored
//    [n][g / 4][hi0..3, lo0..3] with zero padding to a multiple of 4 groups.
__global__ __launch_bounds__(64) void pack_weight_kernel(const uint8_t* __restrict__ qw,
                                                         const uint16_t* __restrict__ sw,
                                                         uint8_t* __restrict__ qwp, int16_t* __restrict__ wsum,
                                                         uint16_t* __restrict__ swp, uint16_t* __restrict__ wcorr,
                                                         float* __restrict__ escale, int* __restrict__ n_neg8,
                                                         int N, int K) {
  const int G = K >> 6, G4 = (G + 3) / 4;
  const int n = blockIdx.x, t = threadIdx.x;
  // row maximum of the (non-negative) weight scales
  float mx = 0.0f;
  for (int g = t; g < G; g += 64) mx = fmaxf(mx, fabsf(f16_bits_to_f32(sw[(int64_t)n * G + g])));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  int e = 0;
  if (mx > 0.0f) e = (int)((__float_as_uint(mx) >> 23) & 0xFF) - 127 - 14;  // f16 values are normal in fp32
  const float down = __uint_as_float((uint32_t)(127 - e) << 23);          // 2^-e, |e| <= 38
  if (t == 0) escale[n] = __uint_as_float((uint32_t)(127 + e) << 23);
  int neg8 = 0;
  for (int g = t; g < 4 * G4; g += 64) {
    float c = 0.0f;
    if (g < G) {
      const uint8_t* src = qw + (int64_t)n * (K >> 1) + g * 32;
      uint8_t* dst = qwp + (int64_t)n * (K >> 1) + g * 32;
      int sum = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t w = *(const uint32_t*)(src + 4 * j);
        uint32_t o = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t by = (w >> (8 * b)) & 0xFFu;
          const int qe = (int)((by & 0xF) ^ 8) - 8;  // element 8j + 2b
          const int qo = (int)((by >> 4) ^ 8) - 8;   // element 8j + 2b + 1
          sum += qe + qo;
          neg8 += (qe == -8) + (qo == -8);
          const uint32_t me = (uint32_t)(qe < 0 ? -qe : qe) & 7u, mo = (uint32_t)(qo < 0 ? -qo : qo) & 7u;
          o |= (me | ((qe < 0 ? 1u : 0u) << 7) | (mo << 4)) << (8 * b);
          o |= (qo < 0 ? 1u : 0u) << (8 * ((b + 1) & 3) + 3);
        }
        *(uint32_t*)(dst + 4 * j) = o;
      }
      wsum[(int64_t)n * G + g] = (int16_t)sum;
      const float swv = f16_bits_to_f32(sw[(int64_t)n * G + g]) * down;
      const uint16_t swb = f32_to_f16_bits(swv);
      swp[(int64_t)n * G + g] = swb;
      c = -(float)sum * f16_bits_to_f32(swb) * (1.0f / 512.0f);
    }
    const uint16_t hi = f32_to_f16_bits(c);
    const uint16_t lo = f32_to_f16_bits(c - f16_bits_to_f32(hi));
    uint16_t* cw = wcorr + ((int64_t)n * G4 + (g >> 2)) * 8;
    cw[g & 3] = hi;
    cw[4 + (g & 3)] = lo;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) neg8 += __shfl_xor(neg8, o);
  if (t == 0 && neg8) atomicAdd(n_neg8, neg8);
}

}  // namespace

extern "C" int gwa_svdq_pack_weight_int4(const uint8_t* qw, const void* sw, uint8_t* qw_packed, int16_t* wsum,
                                         void* sw_packed, void* wcorr, float* escale, int* n_neg8, int64_t N,
                                         int64_t K, void* stream) {
  GWA_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "svdq_pack_weight_int4: bad shape N=%lld K=%lld (K %% 64 == 0)",
              (long long)N, (long long)K);
  GWA_REQUIRE(N < (1ll << 31) && N * (K / 64) < (1ll << 31) && K < (1ll << 30), "svdq_pack_weight_int4: shape too large");
  GWA_REQUIRE(qw && sw && qw_packed && wsum && sw_packed && wcorr && escale && n_neg8,
              "svdq_pack_weight_int4: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qw, 4) && GWA_ALIGNED(qw_packed, 4) && GWA_ALIGNED(wsum, 2) && GWA_ALIGNED(sw, 2) &&
                  GWA_ALIGNED(sw_packed, 2) && GWA_ALIGNED(wcorr, 16) && GWA_ALIGNED(escale, 4) &&
                  GWA_ALIGNED(n_neg8, 4),
              "svdq_pack_weight_int4: misaligned pointer");
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)N), dim3(64), 0, (hipStream_t)stream, qw,
                     (const uint16_t*)sw, qw_packed, wsum, (uint16_t*)sw_packed, (uint16_t*)wcorr, escale, n_neg8,
                     (int)N, (int)K);
  return gwa_check_launch("svdq_pack_weight_int4");
}

extern "C" int gwa_svdq_gemm_w4a4_packed(const uint8_t* qa, const void* sa, const uint8_t* qw_packed,
                                         const void* sw_packed, const void* wcorr, const float* escale,
                                         const float* s2, const float* second, int64_t second_numel, const void* la,
                                         const void* up, int64_t rank, const void* bias, void* out, int out_dtype,
                                         int epilogue_flags, int64_t M, int64_t N, int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && N > 0 && K > 0, "svdq_gemm_w4a4_packed: bad shape M=%lld N=%lld K=%lld", (long long)M,
              (long long)N, (long long)K);
  GWA_REQUIRE(K % 256 == 0, "svdq_gemm_w4a4_packed: K=%lld is not a multiple of 256", (long long)K);
  GWA_REQUIRE(N % 16 == 0, "svdq_gemm_w4a4_packed: N=%lld is not a multiple of 16", (long long)N);
  GWA_REQUIRE(out_dtype == GWA_DT_BF16 || out_dtype == GWA_DT_F16, "svdq_gemm_w4a4_packed: out_dtype %d", out_dtype);
  GWA_REQUIRE((la == nullptr) == (up == nullptr), "svdq_gemm_w4a4_packed: la and up must both be given or both NULL");
  const int64_t R = la ? rank : 0;
  GWA_REQUIRE(R == 0 || R == 16 || R == 32 || R == 64 || R == 128,
              "svdq_gemm_w4a4_packed: rank %lld not in {0,16,32,64,128}", (long long)R);
  GWA_REQUIRE(second == nullptr || second_numel == 1 || second_numel == N,
              "svdq_gemm_w4a4_packed: second has %lld values for N=%lld", (long long)second_numel, (long long)N);
  GWA_REQUIRE((epilogue_flags & ~GWA_EPI_GELU_TANH) == 0, "svdq_gemm_w4a4_packed: unknown epilogue flags 0x%x",
              epilogue_flags);
  GWA_REQUIRE(M * (K / 2) < (1ll << 31) && N * (K / 2) < (1ll << 31) && M * N * 2 < (1ll << 31),
              "svdq_gemm_w4a4_packed: operands must stay below 2 GiB (buffer addressing)");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(qa && sa && qw_packed && sw_packed && wcorr && escale && out, "svdq_gemm_w4a4_packed: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qa, 16) && GWA_ALIGNED(qw_packed, 16) && GWA_ALIGNED(la, 16) && GWA_ALIGNED(up, 16) &&
                  GWA_ALIGNED(out, 8) && GWA_ALIGNED(sa, 8) && GWA_ALIGNED(sw_packed, 8) &&
                  GWA_ALIGNED(wcorr, 16) && GWA_ALIGNED(escale, 4) && GWA_ALIGNED(bias, 2) &&
                  GWA_ALIGNED(second, 4) && GWA_ALIGNED(s2, 4),
              "svdq_gemm_w4a4_packed: misaligned pointer");
  const int64_t tiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
  GWA_REQUIRE(tiles < (1ll << 30), "svdq_gemm_w4a4_packed: too many tiles");
  const bool gelu = epilogue_flags & GWA_EPI_GELU_TANH;
  const bool f16 = out_dtype == GWA_DT_F16;
  hipStream_t s = (hipStream_t)stream;
  const int64_t per_xcd = (tiles + kXcds - 1) / kXcds;
  const dim3 grid((unsigned)(per_xcd * kXcds)), block(NTHREADS);
  const size_t lds = (size_t)LDS_TOTAL;
  const int pc = second_numel > 1;
  const uint16_t* sap = (const uint16_t*)sa;
  const uint16_t* swp = (const uint16_t*)sw_packed;
  const uint16_t* wcp = (const uint16_t*)wcorr;
  const uint16_t* lap = (const uint16_t*)la;
  const uint16_t* upp = (const uint16_t*)up;
  const uint16_t* bp = (const uint16_t*)bias;
  uint16_t* op = (uint16_t*)out;
  const int m = (int)M, n = (int)N, k = (int)K;
#define GWA_FP8_LAUNCH(RBV, GL, F16V)                                                                            \
  hipLaunchKernelGGL((w4a4_gemm_fp8_kernel<RBV, GL, F16V>), grid, block, lds, s, qa, sap, qw_packed, swp, wcp, \
                     escale, s2, second, pc, lap, upp, bp, op, m, n, k)
#define GWA_FP8_RB(RBV)                           \
  case RBV:                                       \
    if (gelu) {                                   \
      if (f16) GWA_FP8_LAUNCH(RBV, true, true);   \
      else GWA_FP8_LAUNCH(RBV, true, false);      \
    } else {                                      \
      if (f16) GWA_FP8_LAUNCH(RBV, false, true);  \
      else GWA_FP8_LAUNCH(RBV, false, false);     \
    }                                             \
    break;
  switch (R / 16) {
    GWA_FP8_RB(0)
    GWA_FP8_RB(1)
    GWA_FP8_RB(2)
    GWA_FP8_RB(4)
    GWA_FP8_RB(8)
    default: return gwa_set_error(GWA_ERR_INVALID, "svdq_gemm_w4a4_packed: rank %lld", (long long)R);
  }
#undef GWA_FP8_RB
#undef GWA_FP8_LAUNCH
  return gwa_check_launch("svdq_gemm_w4a4_packed");
}

extern "C" int gwa_svdq_group_psums_packed(const uint8_t* qa, const uint8_t* qw_packed, const int16_t* wsum,
                                           int32_t* out, int64_t M, int64_t N, int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && N >= 0 && K > 0 && K % 64 == 0, "svdq_group_psums_packed: bad shape (K %% 64 == 0)");
  GWA_REQUIRE(M < (1ll << 31) && N < (1ll << 30) && K < (1ll << 30) && M * N * (K / 64) * 4 < (1ll << 31),
              "svdq_group_psums_packed: shape too large (the output must stay below 2 GiB)");
  GWA_REQUIRE((N + 31) / 32 < 65536, "svdq_group_psums_packed: N too large");
  if (M == 0 || N == 0) return GWA_OK;
  GWA_REQUIRE(qa && qw_packed && wsum && out, "svdq_group_psums_packed: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qa, 16) && GWA_ALIGNED(qw_packed, 16) && GWA_ALIGNED(out, 4) && GWA_ALIGNED(wsum, 2),
              "svdq_group_psums_packed: misaligned pointer");
  hipLaunchKernelGGL(w4a4_psums_fp8_kernel, dim3((unsigned)((M + 31) / 32), (unsigned)((N + 31) / 32)), dim3(64), 0,
                     (hipStream_t)stream, qa, qw_packed, wsum, out, (int)M, (int)N, (int)K);
  return gwa_check_launch("svdq_group_psums_packed");
}
