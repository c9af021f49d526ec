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
//    sum_k q_w (q_x + 8) * 2^-12 = (P + 8 * cw) * 2^-12, where P is the
//    group's exact integer dot product and cw = sum_k q_w. Its C input is
//    -cw * 2^-9 (one fp32 per weight row, prepacked), so the MFMA result is
//    exactly P * 2^-12: every term is a multiple of 2^-12 below 2^4, far
//    inside fp32's 24-bit significand.
//
// Per group and 32x32 block the dequant is then
//    S   = sw[n] * sx[m]   (f16 MFMA 32x32x8, one nonzero K slot; exact)
//    acc = fma(P, S, acc)  (16 VALU fma per lane)
// and the epilogue multiplies by 2^12 * s2 * second[n], adds la @ up^T
// (bf16 MFMA), bias, optional GELU, and stores four consecutive n per lane.
//
// Tiling: a 512-thread workgroup owns a 128 (n) x 256 (m) tile; its 8 waves
// form a 2 x 4 grid of 64 x 64 wave tiles (2 x 2 blocks of 32 x 32), two
// waves per SIMD so one wave's MFMAs overlap the other's VALU dequant. Two
// K-groups per LDS stage, double buffered, rows padded to 80 bytes so the
// 16-byte operand reads are bank-conflict free.
#include "gwa_common.h"

namespace {

constexpr int TN = 128, TM = 256;
constexpr int WBN = 2, WBM = 2;
constexpr int WAVES_N = TN / (32 * WBN), WAVES_M = TM / (32 * WBM);
constexpr int NTHREADS = 64 * WAVES_N * WAVES_M;  // 512
constexpr int GS = 2;                              // groups per stage
constexpr int KTB = GS * 32;                       // packed bytes per row per stage
constexpr int STR = KTB + 16;                      // padded LDS row stride
constexpr int LDS_W = TN * STR, LDS_X = TM * STR;
constexpr int LDS_SW = TN * GS * 2, LDS_SX = TM * GS * 2, LDS_CW = GS * TN * 4;
constexpr int LDS_STAGE = LDS_W + LDS_X + LDS_SW + LDS_SX + LDS_CW;
constexpr int XLOADS = TM * KTB / 16 / NTHREADS;   // 2
static_assert(TN * KTB / 16 == NTHREADS, "one 16-byte weight load per thread per stage");
constexpr int kWScaleE8M0 = 127 + 6;               // 2^6 on the weight operand
constexpr float kUnscale = 4096.0f;                // 2^12

__device__ __forceinline__ uint32_t rotr4(uint32_t w) { return __builtin_amdgcn_alignbit(w, w, 4); }

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

__device__ __forceinline__ v8i act_fp8(v4i p) {
  v8i r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t t = (uint32_t)p[j] ^ 0x88888888u;
    r[j] = (int)(t & 0x0F0F0F0Fu);
    r[4 + j] = (int)((t >> 4) & 0x0F0F0F0Fu);
  }
  return r;
}

// P * 2^-12 for one group: A = weight rows, B = activation rows, C = -cw * 2^-9
__device__ __forceinline__ v16f group_mfma_fp8(v8i a, v8i b, v16f c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, kWScaleE8M0, 0, 127);
}

__device__ __forceinline__ v4h scale_operand(uint16_t s_bits, int h) {
  v4h r = {(_Float16)0, (_Float16)0, (_Float16)0, (_Float16)0};
  if (h == 0) r[0] = __builtin_bit_cast(_Float16, s_bits);
  return r;
}

struct Stage {
  v4i w;
  v4i x[XLOADS];
  uint32_t s;  // two fp16 scales or two int16 column sums, by thread role
};

template <int RB, bool GELU, bool OUT_F16>
__global__ __launch_bounds__(NTHREADS, 1) void w4a4_gemm_fp8_kernel(
    const uint8_t* __restrict__ qa, const uint16_t* __restrict__ sa, const uint8_t* __restrict__ qwp,
    const uint16_t* __restrict__ sw, const int16_t* __restrict__ wsum, const float* __restrict__ s2p,
    const float* __restrict__ second, int second_per_channel, const uint16_t* __restrict__ la,
    const uint16_t* __restrict__ up, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N,
    int K) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x;
  const int tiles_n = (N + TN - 1) / TN;
  const int tn = blockIdx.x % tiles_n, tm = blockIdx.x / tiles_n;
  const int n0 = tn * TN, m0 = tm * TM;
  const int kbytes = K >> 1, G = K >> 6;
  const int nstages = G / GS;
  const int wave = tid >> 6, lane = tid & 63;
  const int wn = wave % WAVES_N, wm = wave / WAVES_N;
  const int r32 = lane & 31, h = lane >> 5;

  const rsrc_t wbuf = make_rsrc(qwp, (uint32_t)((int64_t)N * kbytes));
  const rsrc_t xbuf = make_rsrc(qa, (uint32_t)((int64_t)M * kbytes));
  const rsrc_t swbuf = make_rsrc(sw, (uint32_t)((int64_t)N * G * 2));
  const rsrc_t sxbuf = make_rsrc(sa, (uint32_t)((int64_t)M * G * 2));
  const rsrc_t cwbuf = make_rsrc(wsum, (uint32_t)((int64_t)N * G * 2));

  // loader roles
  const int wrow = tid >> 2, wchunk = tid & 3;
  const uint32_t woff = (uint32_t)((int64_t)(n0 + wrow) * kbytes + wchunk * 16);
  uint32_t xoff[XLOADS];
  int xrow[XLOADS], xchunk[XLOADS];
#pragma unroll
  for (int j = 0; j < XLOADS; ++j) {
    const int idx = tid + j * NTHREADS;
    xrow[j] = idx >> 2;
    xchunk[j] = idx & 3;
    xoff[j] = (uint32_t)((int64_t)(m0 + xrow[j]) * kbytes + xchunk[j] * 16);
  }
  // scale / column-sum loader: 0..127 weight scales, 128..383 activation scales, 384..511 column sums
  const int srole = tid < TN ? 0 : (tid < TN + TM ? 1 : 2);
  const int srow = srole == 0 ? tid : (srole == 1 ? tid - TN : tid - TN - TM);
  const rsrc_t sbuf = srole == 0 ? swbuf : (srole == 1 ? sxbuf : cwbuf);
  const uint32_t soff = (uint32_t)((int64_t)((srole == 1 ? m0 : n0) + srow) * G * 2);

  auto load = [&](Stage& r, int st) {
    r.w = buf_load16(wbuf, woff + st * KTB);
#pragma unroll
    for (int j = 0; j < XLOADS; ++j) r.x[j] = buf_load16(xbuf, xoff[j] + st * KTB);
    r.s = buf_load4(sbuf, soff + st * GS * 2);
  };
  auto store = [&](const Stage& r, int buf) {
    uint8_t* base = lds + buf * LDS_STAGE;
    *(v4i*)(base + wrow * STR + wchunk * 16) = r.w;
#pragma unroll
    for (int j = 0; j < XLOADS; ++j) *(v4i*)(base + LDS_W + xrow[j] * STR + xchunk[j] * 16) = r.x[j];
    if (srole == 0) {
      *(uint32_t*)(base + LDS_W + LDS_X + srow * 4) = r.s;
    } else if (srole == 1) {
      *(uint32_t*)(base + LDS_W + LDS_X + LDS_SW + srow * 4) = r.s;
    } else {
      float* cw = (float*)(base + LDS_W + LDS_X + LDS_SW + LDS_SX);
      cw[srow] = -(float)(int16_t)(r.s & 0xFFFFu) * (1.0f / 512.0f);
      cw[TN + srow] = -(float)(int16_t)(r.s >> 16) * (1.0f / 512.0f);
    }
  };

  v16f acc[WBN][WBM];
#pragma unroll
  for (int a = 0; a < WBN; ++a)
#pragma unroll
    for (int b = 0; b < WBM; ++b) acc[a][b] = (v16f){};

  Stage regs;
  load(regs, 0);
  store(regs, 0);
  __syncthreads();

  for (int st = 0; st < nstages; ++st) {
    const int buf = st & 1;
    if (st + 1 < nstages) load(regs, st + 1);
    const uint8_t* base = lds + buf * LDS_STAGE;
    const uint8_t* lw = base;
    const uint8_t* lx = base + LDS_W;
    const uint16_t* lsw = (const uint16_t*)(base + LDS_W + LDS_X);
    const uint16_t* lsx = (const uint16_t*)(base + LDS_W + LDS_X + LDS_SW);
    const float* lcw = (const float*)(base + LDS_W + LDS_X + LDS_SW + LDS_SX);
#pragma unroll 1
    for (int gi = 0; gi < GS; ++gi) {
      v8i bx[WBM];
      v4h bs[WBM];
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm) {
        const int row = 32 * (WBM * wm + bm) + r32;
        bx[bm] = act_fp8(*(const v4i*)(lx + row * STR + gi * 32 + 16 * h));
        bs[bm] = scale_operand(lsx[row * GS + gi], h);
      }
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn) {
        const int nrow = 32 * (WBN * wn + bn);
        const v8i aw = wgt_fp8(*(const v4i*)(lw + (nrow + r32) * STR + gi * 32 + 16 * h));
        const v4h as = scale_operand(lsw[(nrow + r32) * GS + gi], h);
        v16f dc;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const v4f c4 = *(const v4f*)(lcw + gi * TN + nrow + 8 * q + 4 * h);
          dc[4 * q] = c4[0];
          dc[4 * q + 1] = c4[1];
          dc[4 * q + 2] = c4[2];
          dc[4 * q + 3] = c4[3];
        }
#pragma unroll
        for (int bm = 0; bm < WBM; ++bm) {
          const v16f p = group_mfma_fp8(aw, bx[bm], dc);
          const v16f s = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs[bm], (v16f){}, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[bn][bm][v] = fmaf(p[v], s[v], acc[bn][bm][v]);
        }
      }
    }
    if (st + 1 < nstages) store(regs, buf ^ 1);
    __syncthreads();
  }

  // ---------------- epilogue ----------------
  const rsrc_t obuf = make_rsrc(out, (uint32_t)((int64_t)M * N * 2));
  const float s2 = s2p ? *s2p : 1.0f;
  const float base_mult = s2 * kUnscale;
#pragma unroll
  for (int bn = 0; bn < WBN; ++bn) {
    const int nb = n0 + 32 * (WBN * wn + bn);
#pragma unroll
    for (int bm = 0; bm < WBM; ++bm) {
      const int m = m0 + 32 * (WBM * wm + bm) + r32;
      v16f y = acc[bn][bm];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int n = nb + 8 * (v >> 2) + 4 * h + (v & 3);
        float sec = 1.0f;
        if (second) sec = second[second_per_channel ? (n < N ? n : 0) : 0];
        y[v] *= base_mult * sec;
      }
      if (RB > 0) {
        const int nrow = nb + r32;
        const bool nin = nrow < N, min_ = m < M;
#pragma unroll
        for (int kk = 0; kk < RB; ++kk) {
          const int r0 = kk * 16 + 8 * h;
          v4i ua = nin ? *(const v4i*)(up + (int64_t)nrow * (RB * 16) + r0) : (v4i){0, 0, 0, 0};
          v4i lb = min_ ? *(const v4i*)(la + (int64_t)m * (RB * 16) + r0) : (v4i){0, 0, 0, 0};
          y = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ua), __builtin_bit_cast(v8bf, lb),
                                                      y, 0, 0, 0);
        }
      }
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int n = nb + 8 * qd + 4 * h;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = y[4 * qd + e];
          if (bias) t += bf16_to_f32(bias[n + e < N ? n + e : 0]);
          if (GELU) t = gelu_tanh_f32(t);
          o[e] = t;
        }
        uint2 pk;
        if (OUT_F16) {
          pk.x = pack_f16x2(o[0], o[1]);
          pk.y = pack_f16x2(o[2], o[3]);
        } else {
          pk.x = pack_bf16x2(o[0], o[1]);
          pk.y = pack_bf16x2(o[2], o[3]);
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

// Prepack: logical two's-complement codes -> rotated sign-magnitude layout,
// plus the per-(row, group) code sums. One thread per (row, group).
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint8_t* __restrict__ qw, uint8_t* __restrict__ qwp,
                                                          int16_t* __restrict__ wsum, int* __restrict__ n_neg8,
                                                          int N, int K) {
  const int G = K >> 6;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)N * G) return;
  const int n = (int)(idx / G), g = (int)(idx % G);
  const uint8_t* src = qw + (int64_t)n * (K >> 1) + g * 32;
  uint8_t* dst = qwp + (int64_t)n * (K >> 1) + g * 32;
  int sum = 0, neg8 = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w = *(const uint32_t*)(src + 4 * j);
    uint32_t o = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t by = (w >> (8 * b)) & 0xFFu;
      const int qe = (int)((by & 0xF) ^ 8) - 8;       // element 8j + 2b
      const int qo = (int)((by >> 4) ^ 8) - 8;        // element 8j + 2b + 1
      sum += qe + qo;
      neg8 += (qe == -8) + (qo == -8);
      const uint32_t me = (uint32_t)(qe < 0 ? -qe : qe) & 7u, mo = (uint32_t)(qo < 0 ? -qo : qo) & 7u;
      o |= (me | ((qe < 0 ? 1u : 0u) << 7) | (mo << 4)) << (8 * b);
      o |= (qo < 0 ? 1u : 0u) << (8 * ((b + 1) & 3) + 3);
    }
    *(uint32_t*)(dst + 4 * j) = o;
  }
  wsum[idx] = (int16_t)sum;
  if (neg8) atomicAdd(n_neg8, neg8);
}

}  // namespace

extern "C" int gwa_svdq_pack_weight_int4(const uint8_t* qw, uint8_t* qw_packed, int16_t* wsum, int* n_neg8,
                                         int64_t N, int64_t K, void* stream) {
  GWA_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "svdq_pack_weight_int4: bad shape N=%lld K=%lld (K %% 64 == 0)",
              (long long)N, (long long)K);
  GWA_REQUIRE(N * (K / 64) < (1ll << 31) && K < (1ll << 30), "svdq_pack_weight_int4: shape too large");
  GWA_REQUIRE(qw && qw_packed && wsum && n_neg8, "svdq_pack_weight_int4: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qw, 4) && GWA_ALIGNED(qw_packed, 4) && GWA_ALIGNED(wsum, 2) && GWA_ALIGNED(n_neg8, 4),
              "svdq_pack_weight_int4: misaligned pointer");
  const int64_t total = N * (K / 64);
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     qw, qw_packed, wsum, n_neg8, (int)N, (int)K);
  return gwa_check_launch("svdq_pack_weight_int4");
}

extern "C" int gwa_svdq_gemm_w4a4_packed(const uint8_t* qa, const void* sa, const uint8_t* qw_packed,
                                         const void* sw, const int16_t* wsum, const float* s2, const float* second,
                                         int64_t second_numel, const void* la, const void* up, int64_t rank,
                                         const void* bias, void* out, int out_dtype, int epilogue_flags, int64_t M,
                                         int64_t N, int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && N > 0 && K > 0, "svdq_gemm_w4a4_packed: bad shape M=%lld N=%lld K=%lld", (long long)M,
              (long long)N, (long long)K);
  GWA_REQUIRE(K % 128 == 0, "svdq_gemm_w4a4_packed: K=%lld is not a multiple of 128", (long long)K);
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
  GWA_REQUIRE(qa && sa && qw_packed && sw && wsum && out, "svdq_gemm_w4a4_packed: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qa, 16) && GWA_ALIGNED(qw_packed, 16) && GWA_ALIGNED(la, 16) && GWA_ALIGNED(up, 16) &&
                  GWA_ALIGNED(out, 8) && GWA_ALIGNED(sa, 4) && GWA_ALIGNED(sw, 4) && GWA_ALIGNED(wsum, 4) &&
                  GWA_ALIGNED(bias, 2) && GWA_ALIGNED(second, 4) && GWA_ALIGNED(s2, 4),
              "svdq_gemm_w4a4_packed: misaligned pointer");
  const int64_t tiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
  GWA_REQUIRE(tiles < (1ll << 31), "svdq_gemm_w4a4_packed: too many tiles");
  const bool gelu = epilogue_flags & GWA_EPI_GELU_TANH;
  const bool f16 = out_dtype == GWA_DT_F16;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)tiles), block(NTHREADS);
  const size_t lds = 2 * (size_t)LDS_STAGE;
  const int pc = second_numel > 1;
  const uint16_t* sap = (const uint16_t*)sa;
  const uint16_t* swp = (const uint16_t*)sw;
  const uint16_t* lap = (const uint16_t*)la;
  const uint16_t* upp = (const uint16_t*)up;
  const uint16_t* bp = (const uint16_t*)bias;
  uint16_t* op = (uint16_t*)out;
  const int m = (int)M, n = (int)N, k = (int)K;
#define GWA_FP8_LAUNCH(RBV, GL, F16V)                                                                          \
  hipLaunchKernelGGL((w4a4_gemm_fp8_kernel<RBV, GL, F16V>), grid, block, lds, s, qa, sap, qw_packed, swp, wsum, s2, \
                     second, pc, lap, upp, bp, op, m, n, k)
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
