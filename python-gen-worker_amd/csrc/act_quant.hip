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
// Output formats: GWA_QFMT_INT4 is the reference contract (two's-complement
// nibbles, element 2j in the low nibble of byte j); GWA_QFMT_FP6 writes the
// same codes as e3m2 fp6 in the fp6 GEMM's operand records (one 104-byte
// record per 128-column stage and row, stage-major: 96 bytes of codes with
// element t of a group at bits [6t, 6t+6) of the group's 48 bytes, then the
// stage's two fp16 group scales).
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

template <int RB, int FMT, int PF>
__global__ __launch_bounds__(512) void svdq_quant_int4_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ smooth,
    const float* __restrict__ s2p, const uint16_t* __restrict__ pdo, uint8_t* __restrict__ q,
    uint16_t* __restrict__ sc, void* __restrict__ la, int la_f32_add, int M, int K) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int RBX = RB > 0 ? RB : 1;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int row0 = blockIdx.x * 16;
  const int G = K >> 6;
  const int rounds = (K + KT - 1) / KT;

  // buffers: every access is unconditional; rows >= M, columns >= K read 0 / store nothing
  const rsrc_t xbuf = make_rsrc(x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2));
  // FP6: [K/128][M][104] records (96 bytes of codes, 2 fp16 scales, 4 unused bytes)
  const int64_t qrow_bytes = FMT == GWA_QFMT_FP6 ? (int64_t)(K / 128) * GWA_FP6_REC : (int64_t)K / 2;
  const rsrc_t qbuf = make_rsrc(q, (uint32_t)((int64_t)M * qrow_bytes));
  const rsrc_t sbuf = make_rsrc(sc, sc ? (uint32_t)((int64_t)M * G * 2) : 0u);
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
        const bool valid = kg < K && grow < M;  // rows past M must not store (fp6 records of the next stage follow)
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
        if (FMT == GWA_QFMT_FP6) {
          // record of (128-column stage g / 2, row), group g % 2 of the stage
          const uint32_t rec = (uint32_t)(((int64_t)(g >> 1) * M + grow) * GWA_FP6_REC);
          g64::store_fp6(qbuf, rec, g & 1, lane, nb, sh, valid);
        } else {
          const uint32_t a = nb[0], bb = nb[1];
          const uint32_t pa = (a & 0xFu) | ((a >> 4) & 0xF0u) | ((a >> 8) & 0xF00u) | ((a >> 12) & 0xF000u);
          const uint32_t pb = (bb & 0xFu) | ((bb >> 4) & 0xF0u) | ((bb >> 8) & 0xF00u) | ((bb >> 12) & 0xF000u);
          buf_store4(pa | (pb << 16), qbuf, valid ? q_row_off + (uint32_t)(kg / 2) : kOOB);
        }
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
    // sum the 8 waves' partial la blocks through LDS; wave 0 writes bf16 (or adds into fp32)
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
          if (r < M) {
            const int64_t i = (int64_t)r * R + rb * 16 + (lane & 15);
            if (la_f32_add) ((float*)la)[i] += s[t];  // rows are this workgroup's alone
            else ((uint16_t*)la)[i] = f32_to_bf16(s[t]);
          }
        }
      }
    }
  }
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
// int8 per-token quantization: one 256-thread block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void w8a8_quant_int8_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                              int8_t* __restrict__ q, float* __restrict__ sa,
                                                              int M, int K) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const uint16_t* xr = x + (int64_t)row * ldx;
  int8_t* qr = q + (int64_t)row * K;
  const int nchunk = K >> 3;
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
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(am / 127.0f, 1e-12f);
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
  if (threadIdx.x == 0) sa[row] = s;
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

static int quant_int4(const void* x, int64_t ldx, const void* smooth, const float* s2, const void* proj_down_op,
                      int64_t rank, int out_format, uint8_t* q, void* scales, void* la, int la_f32_add, int64_t M,
                      int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && K > 0, "svdq_quant_int4: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  GWA_REQUIRE(K % 64 == 0, "svdq_quant_int4: K=%lld is not a multiple of 64", (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "svdq_quant_int4: row stride %lld must be >= K and a multiple of 8",
              (long long)ldx);
  GWA_REQUIRE(out_format == GWA_QFMT_INT4 || out_format == GWA_QFMT_FP6, "svdq_quant_int4: out_format %d",
              out_format);
  GWA_REQUIRE(out_format != GWA_QFMT_FP6 || K % 128 == 0, "svdq_quant_int4: the fp6 format needs K %% 128 == 0 (K=%lld)",
              (long long)K);
  GWA_REQUIRE((proj_down_op == nullptr) == (la == nullptr),
              "svdq_quant_int4: proj_down_op and la must both be given or both be NULL");
  const int64_t R = proj_down_op ? rank : 0;
  GWA_REQUIRE(R == 0 || R == 16 || R == 32 || R == 64 || R == 128,
              "svdq_quant_int4: rank %lld not in {0,16,32,64,128}", (long long)R);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 24) && (M * ldx * 2) < (1ll << 31) &&
                  M * (K / 128) * GWA_FP6_REC < (1ll << 31),
              "svdq_quant_int4: x and q must stay below 2 GiB (buffer addressing)");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && q && (scales || out_format == GWA_QFMT_FP6), "svdq_quant_int4: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q, out_format == GWA_QFMT_FP6 ? 8 : 16) && GWA_ALIGNED(scales, 2) && GWA_ALIGNED(smooth, 4) &&
                  GWA_ALIGNED(proj_down_op, 16) && GWA_ALIGNED(la, la_f32_add ? 4 : 2),
              "svdq_quant_int4: x and proj_down_op must be 16-byte aligned, q 16 (int4) or 8 (fp6)");
  hipStream_t s = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  const uint16_t* sm = (const uint16_t*)smooth;
  const uint16_t* pd = (const uint16_t*)proj_down_op;
  uint16_t* sc = (uint16_t*)scales;
  void* lp = la;
  const int m = (int)M, k = (int)K;
  const int rb = (int)(R / 16);
  const size_t lds = 2 * (size_t)QBUF > (size_t)rb * 8192 ? 2 * (size_t)QBUF : (size_t)rb * 8192;
  const dim3 grid((unsigned)((M + 15) / 16)), block(512);
  const bool fp6 = out_format == GWA_QFMT_FP6;
#define GWA_QUANT_LAUNCH(RBV, PFV)                                                                               \
  if (fp6)                                                                                                       \
    hipLaunchKernelGGL((svdq_quant_int4_kernel<RBV, GWA_QFMT_FP6, PFV>), grid, block, lds, s, xp, ldx, sm, s2, pd, \
                       q, sc, lp, la_f32_add, m, k);                                                              \
  else                                                                                                           \
    hipLaunchKernelGGL((svdq_quant_int4_kernel<RBV, GWA_QFMT_INT4, PFV>), grid, block, lds, s, xp, ldx, sm, s2,   \
                       pd, q, sc, lp, la_f32_add, m, k);
  switch (rb) {
    case 0: GWA_QUANT_LAUNCH(0, 4) break;
    case 1: GWA_QUANT_LAUNCH(1, 4) break;
    case 2: GWA_QUANT_LAUNCH(2, 4) break;
    case 4: GWA_QUANT_LAUNCH(4, 3) break;
    case 8: GWA_QUANT_LAUNCH(8, 2) break;
    default: return gwa_set_error(GWA_ERR_INVALID, "svdq_quant_int4: rank %lld not in {0,16,32,64,128}", (long long)R);
  }
#undef GWA_QUANT_LAUNCH
  return gwa_check_launch("svdq_quant_int4");
}

extern "C" int gwa_svdq_quant_int4(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                   const void* proj_down_op, int64_t rank, int out_format, uint8_t* q,
                                   void* scales, void* la, int64_t M, int64_t K, void* stream) {
  return quant_int4(x, ldx, smooth, s2, proj_down_op, rank, out_format, q, scales, la, 0, M, K, stream);
}

extern "C" int gwa_svdq_quant_fp6_la_f32(const void* x, int64_t ldx, const void* smooth, const void* proj_down_op,
                                         int64_t rank, uint8_t* q6, float* la32, int64_t M, int64_t K,
                                         void* stream) {
  return quant_int4(x, ldx, smooth, nullptr, proj_down_op, rank, GWA_QFMT_FP6, q6, nullptr, la32, 1, M, K, stream);
}

extern "C" int gwa_w8a8_quant_int8(const void* x, int64_t ldx, int8_t* q, float* sa, int64_t M, int64_t K,
                                   void* stream) {
  GWA_REQUIRE(M >= 0 && K > 0 && K % 8 == 0, "w8a8_quant_int8: bad shape M=%lld K=%lld (K %% 8 == 0)",
              (long long)M, (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "w8a8_quant_int8: bad row stride %lld", (long long)ldx);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 30), "w8a8_quant_int8: shape too large");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && q && sa, "w8a8_quant_int8: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q, 8) && GWA_ALIGNED(sa, 4),
              "w8a8_quant_int8: x must be 16-byte and q 8-byte aligned");
  hipLaunchKernelGGL(w8a8_quant_int8_kernel, dim3((unsigned)M), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, ldx, q, sa, (int)M, (int)K);
  return gwa_check_launch("w8a8_quant_int8");
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
