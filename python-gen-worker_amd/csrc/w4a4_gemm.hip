// W4A4 GEMM with per-group dequant and the fused SVDQuant epilogue (gfx950).
//
// Orientation: the MFMA "A" operand is the weight tile (rows n), the "B"
// operand is the activation tile (rows m), so a 32x32 accumulator block is
// D[n][m]; lane l holds column m = l % 32 and rows
// n = 8*(v/4) + 4*(l/32) + (v%4), v = 0..15 — four consecutive n per
// quad, which makes every output store an 8-byte [m, n..n+3] write.
//
// Per K-group of 64 and per 32x32 block:
//   P  = two int8 MFMA 32x32x32 on nibble-in-high-half bytes (= 16*q), so
//        P = 256 * sum_{k in g} qx*qw exactly (int32);
//   S  = sw[n] * sx[m] from one f16 MFMA 32x32x8 with a single nonzero K
//        slot (fp16 x fp16 products are exact in fp32);
//   acc += float(P) * S.
// The 1/256 is folded into the epilogue multiplier.
#include "gwa_common.h"

namespace {

constexpr int TILE = 128;          // block tile: 128 (n) x 128 (m), 4 waves as 2 x 2
constexpr int KT = 128;            // packed bytes per row per stage = 4 groups of 64 codes
constexpr int GPS = KT / 32;       // groups per stage
constexpr int LDS_STRIDE = KT + 16;  // padded row stride (bytes): conflict-free 16B reads
constexpr int LDS_TILE = TILE * LDS_STRIDE;
constexpr int LOADS = TILE * KT / 16 / 256;  // 16B loads per thread per operand per stage

struct StageRegs {
  v4i w[LOADS];
  v4i x[LOADS];
  uint16_t sc[GPS];  // threads 0..127: weight scales of row t; 128..255: activation scales
};

__device__ __forceinline__ void load_stage(StageRegs& r, const uint8_t* __restrict__ qw,
                                           const uint8_t* __restrict__ qa, const uint16_t* __restrict__ sw,
                                           const uint16_t* __restrict__ sa, int n0, int m0, int N, int M,
                                           int kbytes, int G, int stage) {
  const int t = threadIdx.x;
  const int kb0 = stage * KT;
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int idx = t + j * 256;
    const int row = idx / (KT / 16), c = idx % (KT / 16);
    const int kb = kb0 + c * 16;
    const bool kin = kb < kbytes;
    r.w[j] = (n0 + row < N && kin) ? *(const v4i*)(qw + (int64_t)(n0 + row) * kbytes + kb) : (v4i){0, 0, 0, 0};
    r.x[j] = (m0 + row < M && kin) ? *(const v4i*)(qa + (int64_t)(m0 + row) * kbytes + kb) : (v4i){0, 0, 0, 0};
  }
  const int row = t & (TILE - 1);
  const bool is_w = t < TILE;
  const int grow = (is_w ? n0 : m0) + row;
  const bool rin = grow < (is_w ? N : M);
  const uint16_t* src = (is_w ? sw : sa) + (int64_t)grow * G;
#pragma unroll
  for (int j = 0; j < GPS; ++j) {
    const int g = stage * GPS + j;
    r.sc[j] = (rin && g < G) ? src[g] : (uint16_t)0;
  }
}

__device__ __forceinline__ void store_stage(const StageRegs& r, uint8_t* lw, uint8_t* lx, uint16_t* lsc) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int idx = t + j * 256;
    const int row = idx / (KT / 16), c = idx % (KT / 16);
    *(v4i*)(lw + row * LDS_STRIDE + c * 16) = r.w[j];
    *(v4i*)(lx + row * LDS_STRIDE + c * 16) = r.x[j];
  }
  // scale tile: [2][TILE][GPS] fp16 (0 = weights, 1 = activations)
#pragma unroll
  for (int j = 0; j < GPS; ++j) lsc[t * GPS + j] = r.sc[j];
}

// 256 * sum over one K-group, from 16 packed bytes per lane of each operand.
__device__ __forceinline__ v16i group_mfma_i8(v4i a, v4i b) {
  v4i alo, ahi, blo, bhi;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    alo[j] = (int)int4_lo_x16((uint32_t)a[j]);
    ahi[j] = (int)int4_hi_x16((uint32_t)a[j]);
    blo[j] = (int)int4_lo_x16((uint32_t)b[j]);
    bhi[j] = (int)int4_hi_x16((uint32_t)b[j]);
  }
  v16i p = {};
  p = __builtin_amdgcn_mfma_i32_32x32x32_i8(alo, blo, p, 0, 0, 0);
  p = __builtin_amdgcn_mfma_i32_32x32x32_i8(ahi, bhi, p, 0, 0, 0);
  return p;
}

// A-operand (or B-operand) of the f16 scale-product MFMA: only K slot 0 of
// lanes 0..31 is nonzero.
__device__ __forceinline__ v4h scale_operand(uint16_t s_bits, int h) {
  v4h r = {(_Float16)0, (_Float16)0, (_Float16)0, (_Float16)0};
  if (h == 0) r[0] = __builtin_bit_cast(_Float16, s_bits);
  return r;
}

template <int RB, bool GELU, bool OUT_F16>
__global__ __launch_bounds__(256) void w4a4_gemm_kernel(
    const uint8_t* __restrict__ qa, const uint16_t* __restrict__ sa, const uint8_t* __restrict__ qw,
    const uint16_t* __restrict__ sw, const float* __restrict__ s2p, const float* __restrict__ second,
    int second_per_channel, const uint16_t* __restrict__ la, const uint16_t* __restrict__ up,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[2][LDS_TILE];
  __shared__ __attribute__((aligned(16))) uint8_t lds_x[2][LDS_TILE];
  __shared__ uint16_t lds_sc[2][2 * TILE * GPS];

  const int tiles_n = (N + TILE - 1) / TILE;
  const int tn = blockIdx.x % tiles_n, tm = blockIdx.x / tiles_n;
  const int n0 = tn * TILE, m0 = tm * TILE;
  const int kbytes = K >> 1, G = K >> 6;
  const int nstages = (kbytes + KT - 1) / KT;

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wn = wave & 1, wm = wave >> 1;
  const int r32 = lane & 31, h = lane >> 5;

  v16f acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = (v16f){};

  StageRegs regs;
  load_stage(regs, qw, qa, sw, sa, n0, m0, N, M, kbytes, G, 0);
  store_stage(regs, lds_w[0], lds_x[0], lds_sc[0]);
  __syncthreads();

  for (int st = 0; st < nstages; ++st) {
    const int buf = st & 1;
    if (st + 1 < nstages) load_stage(regs, qw, qa, sw, sa, n0, m0, N, M, kbytes, G, st + 1);

    const uint8_t* lw = lds_w[buf];
    const uint8_t* lx = lds_x[buf];
    const uint16_t* lsc = lds_sc[buf];
#pragma unroll 1
    for (int gi = 0; gi < GPS; ++gi) {
      v4i a[2], b[2];
      v4h as[2], bs[2];
#pragma unroll
      for (int bn = 0; bn < 2; ++bn) {
        const int row = 64 * wn + 32 * bn + r32;
        a[bn] = *(const v4i*)(lw + row * LDS_STRIDE + gi * 32 + 16 * h);
        as[bn] = scale_operand(lsc[row * GPS + gi], h);
      }
#pragma unroll
      for (int bm = 0; bm < 2; ++bm) {
        const int row = 64 * wm + 32 * bm + r32;
        b[bm] = *(const v4i*)(lx + row * LDS_STRIDE + gi * 32 + 16 * h);
        bs[bm] = scale_operand(lsc[(TILE + row) * GPS + gi], h);
      }
#pragma unroll
      for (int bn = 0; bn < 2; ++bn) {
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) {
          const v16i p = group_mfma_i8(a[bn], b[bm]);
          const v16f s = __builtin_amdgcn_mfma_f32_32x32x8f16(as[bn], bs[bm], (v16f){}, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[bn][bm][v] = fmaf((float)p[v], s[v], acc[bn][bm][v]);
        }
      }
    }

    if (st + 1 < nstages) {
      store_stage(regs, lds_w[buf ^ 1], lds_x[buf ^ 1], lds_sc[buf ^ 1]);
    }
    __syncthreads();
  }

  // ---------------- epilogue ----------------
  const rsrc_t obuf = make_rsrc(out, (uint32_t)((int64_t)M * N * 2));
  const float s2 = s2p ? *s2p : 1.0f;
  const float base_mult = s2 * (1.0f / 256.0f);
#pragma unroll
  for (int bn = 0; bn < 2; ++bn) {
    const int nb = n0 + 64 * wn + 32 * bn;
#pragma unroll
    for (int bm = 0; bm < 2; ++bm) {
      const int m = m0 + 64 * wm + 32 * bm + r32;
      v16f y = acc[bn][bm];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int n = nb + 8 * (v >> 2) + 4 * h + (v & 3);
        float sec = 1.0f;
        if (second) sec = second[second_per_channel ? (n < N ? n : 0) : 0];
        y[v] *= base_mult * sec;
      }
      if (RB > 0) {
        // low-rank up-projection: D[n][m] += sum_r up[n][r] * la[m][r], bf16 MFMA 32x32x16
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

// Debug: exact per-group int32 partial sums, one wave per 32x32 block.
__global__ __launch_bounds__(64) void w4a4_psums_kernel(const uint8_t* __restrict__ qa,
                                                        const uint8_t* __restrict__ qw,
                                                        int32_t* __restrict__ out, int M, int N, int K) {
  const int lane = threadIdx.x, r32 = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
  const int kbytes = K >> 1, G = K >> 6;
  const int m = m0 + r32, nr = n0 + r32;
  const rsrc_t obuf = make_rsrc(out, (uint32_t)((int64_t)M * N * G * 4));
  for (int g = 0; g < G; ++g) {
    v4i a = nr < N ? *(const v4i*)(qw + (int64_t)nr * kbytes + g * 32 + 16 * h) : (v4i){0, 0, 0, 0};
    v4i b = m < M ? *(const v4i*)(qa + (int64_t)m * kbytes + g * 32 + 16 * h) : (v4i){0, 0, 0, 0};
    const v16i p = group_mfma_i8(a, b);
    // branch-free stores (see the fp8 path): the buffer bounds drop the tails
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int n = n0 + 8 * (v >> 2) + 4 * h + (v & 3);
      const uint32_t off = (m < M && n < N) ? (uint32_t)((((int64_t)m * N + n) * G + g) * 4) : kOOB;
      buf_store4((uint32_t)(p[v] >> 8), obuf, off);
    }
  }
}

}  // namespace

extern "C" int gwa_svdq_gemm_w4a4(const uint8_t* qa, const void* sa, const uint8_t* qw, const void* sw,
                                  const float* s2, const float* second, int64_t second_numel, const void* la,
                                  const void* up, int64_t rank, const void* bias, void* out, int out_dtype,
                                  int epilogue_flags, int64_t M, int64_t N, int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && N > 0 && K > 0, "svdq_gemm_w4a4: bad shape M=%lld N=%lld K=%lld", (long long)M,
              (long long)N, (long long)K);
  GWA_REQUIRE(K % 64 == 0, "svdq_gemm_w4a4: K=%lld is not a multiple of 64", (long long)K);
  GWA_REQUIRE(N % 16 == 0, "svdq_gemm_w4a4: N=%lld is not a multiple of 16", (long long)N);
  GWA_REQUIRE(out_dtype == GWA_DT_BF16 || out_dtype == GWA_DT_F16, "svdq_gemm_w4a4: out_dtype %d not bf16/f16",
              out_dtype);
  GWA_REQUIRE((la == nullptr) == (up == nullptr), "svdq_gemm_w4a4: la and up must both be given or both NULL");
  const int64_t R = la ? rank : 0;
  GWA_REQUIRE(R == 0 || R == 16 || R == 32 || R == 64 || R == 128,
              "svdq_gemm_w4a4: rank %lld not in {0,16,32,64,128}", (long long)R);
  GWA_REQUIRE(second == nullptr || second_numel == 1 || second_numel == N,
              "svdq_gemm_w4a4: second has %lld values for N=%lld", (long long)second_numel, (long long)N);
  GWA_REQUIRE((epilogue_flags & ~GWA_EPI_GELU_TANH) == 0, "svdq_gemm_w4a4: unknown epilogue flags 0x%x",
              epilogue_flags);
  GWA_REQUIRE(M < (1ll << 31) && N < (1ll << 30) && K < (1ll << 30) && M * N * 2 < (1ll << 31),
              "svdq_gemm_w4a4: shape too large (the output must stay below 2 GiB)");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(qa && sa && qw && sw && out, "svdq_gemm_w4a4: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qa, 16) && GWA_ALIGNED(qw, 16) && GWA_ALIGNED(la, 16) && GWA_ALIGNED(up, 16) &&
                  GWA_ALIGNED(out, 8) && GWA_ALIGNED(sa, 2) && GWA_ALIGNED(sw, 2) && GWA_ALIGNED(bias, 2) &&
                  GWA_ALIGNED(second, 4) && GWA_ALIGNED(s2, 4),
              "svdq_gemm_w4a4: qa/qw/la/up must be 16-byte and out 8-byte aligned");
  const int64_t tiles = ((M + TILE - 1) / TILE) * ((N + TILE - 1) / TILE);
  GWA_REQUIRE(tiles < (1ll << 31), "svdq_gemm_w4a4: too many tiles");
  const bool gelu = epilogue_flags & GWA_EPI_GELU_TANH;
  const bool f16 = out_dtype == GWA_DT_F16;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)tiles), block(256);
  const int pc = second_numel > 1;
  const uint16_t* sap = (const uint16_t*)sa;
  const uint16_t* swp = (const uint16_t*)sw;
  const uint16_t* lap = (const uint16_t*)la;
  const uint16_t* upp = (const uint16_t*)up;
  const uint16_t* bp = (const uint16_t*)bias;
  uint16_t* op = (uint16_t*)out;
  const int m = (int)M, n = (int)N, k = (int)K;
#define GWA_W4A4_LAUNCH(RBV, GL, F16V)                                                                      \
  hipLaunchKernelGGL((w4a4_gemm_kernel<RBV, GL, F16V>), grid, block, 0, s, qa, sap, qw, swp, s2, second, pc, \
                     lap, upp, bp, op, m, n, k)
#define GWA_W4A4_RB(RBV)                                   \
  case RBV:                                                \
    if (gelu) {                                            \
      if (f16) GWA_W4A4_LAUNCH(RBV, true, true);           \
      else GWA_W4A4_LAUNCH(RBV, true, false);              \
    } else {                                               \
      if (f16) GWA_W4A4_LAUNCH(RBV, false, true);          \
      else GWA_W4A4_LAUNCH(RBV, false, false);             \
    }                                                      \
    break;
  switch (R / 16) {
    GWA_W4A4_RB(0)
    GWA_W4A4_RB(1)
    GWA_W4A4_RB(2)
    GWA_W4A4_RB(4)
    GWA_W4A4_RB(8)
    default:
      return gwa_set_error(GWA_ERR_INVALID, "svdq_gemm_w4a4: rank %lld not in {0,16,32,64,128}", (long long)R);
  }
#undef GWA_W4A4_RB
#undef GWA_W4A4_LAUNCH
  return gwa_check_launch("svdq_gemm_w4a4");
}

extern "C" int gwa_svdq_group_psums(const uint8_t* qa, const uint8_t* qw, int32_t* out, int64_t M, int64_t N,
                                    int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && N >= 0 && K > 0 && K % 64 == 0, "svdq_group_psums: bad shape (K %% 64 == 0)");
  GWA_REQUIRE(M < (1ll << 31) && N < (1ll << 30) && K < (1ll << 30) && M * N * (K / 64) * 4 < (1ll << 31),
              "svdq_group_psums: shape too large (the output must stay below 2 GiB)");
  GWA_REQUIRE((N + 31) / 32 < 65536, "svdq_group_psums: N too large");
  if (M == 0 || N == 0) return GWA_OK;
  GWA_REQUIRE(qa && qw && out, "svdq_group_psums: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qa, 16) && GWA_ALIGNED(qw, 16) && GWA_ALIGNED(out, 4),
              "svdq_group_psums: qa/qw must be 16-byte aligned");
  hipLaunchKernelGGL(w4a4_psums_kernel, dim3((unsigned)((M + 31) / 32), (unsigned)((N + 31) / 32)), dim3(64), 0,
                     (hipStream_t)stream, qa, qw, out, (int)M, (int)N, (int)K);
  return gwa_check_launch("svdq_group_psums");
}
