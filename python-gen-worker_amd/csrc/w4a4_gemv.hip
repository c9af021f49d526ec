// W4A4 linear for a few tokens (M <= 8): the SVDQuant forward of the reference's fused module
// (_SvdqFusedLinear.forward, models/svdq_fused.py:516-527) at the token counts of the DiT's adaLN modulation
// linears (one token per image). There the GEMM tiles would compute 32 or 128 rows for each real one and
// stream the fp6 weight records (104 bytes per row and 128 inputs) through LDS; this path streams the int4
// weight [N, K/2] (64 bytes per row and 128 inputs, the module's own `weight` buffer) once, straight into
// registers, and takes the integer dot products with v_dot8_i32_i4.
//
// Work split: a 256-thread workgroup owns 32 (or 16) output columns (weight rows) n0 .., i.e. ROWS x G items
// (row, group), G = K / 64; each thread loads its items' 32 weight bytes and fp16 scale first, then
//  1. issues every other load up front (activation rows, smoothing factors, la partial slots), then
//     quantizes the M activation rows itself (every workgroup; M * K is small): the group-64 quantizer of
//     kernel 1 (quant_g64.h quant8: smoothing by RN(1/s), scale RN(amax / 7), RNE codes), so codes and
//     scales are bit-identical to kernel 1's; codes packed 8 nibbles per dword (element i at bits 4i..4i+3,
//     the weight's packing), scales as floats, into LDS;
//  2. sums kernel 1's la partial slots in slot order and rounds to bf16 (la_reduce_kernel's arithmetic);
//     (loaded in one batch: a dependent load per slot cost ~0.8 us each);
//  3. P[m][row][g] = sum of the group's 64 code products (8 x v_dot8_i32_i4, exact) into LDS;
//  4. one lane per (token, row) runs the output's chain in the GEMM's order: acc = fma(P_g, sx_g * sw_g, acc)
//     for g = 0 .. G-1 (sx * sw exact in fp32), acc * (s2 * second[n]), + la . up[n] (fp32 fmas in rank
//     order; the GEMM adds the same products with a bf16 MFMA), + bias, optional GELU-tanh, bf16 / fp16.
//     Without a low-rank term, acc * mult + bias is one fma, as the GEMM's compiled epilogue forms it.
// The accumulation order over groups equals the GEMM's, so the outputs differ from the GEMM lane's only by
// the low-rank sum's rounding (rank 0: bit-identical).
#include "gwa_common.h"
#include "quant_g64.h"

namespace {

// a workgroup owns ROWS = 16 or 32 weight rows; items (row, group) per thread <= GV_MAX_ITEMS
constexpr int GV_THREADS = 256, GV_MAX_M = 8, GV_MAX_ITEMS = 8;

// Dynamic LDS layout (bytes), all float / u32 arrays. Strides are odd numbers of dwords where lanes read
// across them: a group's 8 code dwords sit cs = 9 apart (step 3: lanes on consecutive groups), a row's
// per-group values gp = G + 1 apart (step 4: lanes on consecutive rows), so those reads hit distinct banks
// (at the plain strides of 8 and G = 48 dwords they were 8-way conflicts). A shape whose padded layout would
// pass 64 KB keeps the plain strides (cs = 8, gp = G); host and kernel derive the same layout.
struct GvLds {
  int codes, sx, la, sw, p, total, cs, gp;
  __host__ __device__ void place(int M, int G, int R, int ROWS) {
    codes = 0;                     // u32 [M][G][cs]
    sx = codes + M * G * cs * 4;   // f32 [M][G]
    la = sx + M * G * 4;           // f32 [M][R]
    sw = la + M * R * 4;           // f32 [ROWS][gp]
    p = sw + ROWS * gp * 4;        // f32 [M][ROWS][gp]
    total = p + M * ROWS * gp * 4;
  }
  __host__ __device__ GvLds(int M, int K, int R, int ROWS) {
    const int G = K / 64;
    cs = 9;
    gp = G + 1;
    place(M, G, R, ROWS);
    if (total > 64 * 1024) {
      cs = 8;
      gp = G;
      place(M, G, R, ROWS);
    }
  }
};
// The footprint the token limit and the row count are chosen by: the plain layout's.
__host__ __device__ inline int gv_budget_bytes(int M, int K, int R, int ROWS) {
  const int G = K / 64;
  return M * (K / 8) * 4 + M * G * 4 + M * R * 4 + ROWS * G * 4 + M * ROWS * G * 4;
}

// nb[0] = codes of elements 0..3 (one nibble per byte), nb[1] = elements 4..7 -> 8 nibbles, element i at 4i
__device__ __forceinline__ uint32_t pack_nibbles8(const uint32_t nb[2]) {
  const uint32_t a = nb[0] | (nb[0] >> 4), b = nb[1] | (nb[1] >> 4);  // bytes 0, 2: (e0 | e1 << 4), (e2 | e3 << 4)
  return __builtin_amdgcn_perm(b, a, 0x06040200u);                     // a.byte0, a.byte2, b.byte0, b.byte2
}

template <int RB, int GV_ROWS>
__global__ __launch_bounds__(GV_THREADS) void svdq_gemv_w4a4_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ smooth, const float* __restrict__ s2p,
    const float* __restrict__ la_part, int P, const uint8_t* __restrict__ qw, const uint16_t* __restrict__ sw,
    const float* __restrict__ second, int second_per_channel, const uint16_t* __restrict__ up,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int gelu, int out_f16, int M, int N, int K) {
  constexpr int R = RB * 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t gv_lds[];
  const GvLds L(M, K, R, GV_ROWS);
  uint32_t* codes = (uint32_t*)(gv_lds + L.codes);
  float* sxl = (float*)(gv_lds + L.sx);
  float* lal = (float*)(gv_lds + L.la);
  float* swl = (float*)(gv_lds + L.sw);
  float* pl = (float*)(gv_lds + L.p);
  const int tid = threadIdx.x, G = K >> 6, n0 = blockIdx.x * GV_ROWS;
  const int items = GV_ROWS * G;

  // 0. the small, cache-resident reads first (vector loads complete in issue order, so step 2 waits only for
  //    these, and the quantization runs while the weight stream below is in flight): the rows to quantize
  //    and their smoothing factors (the first QPRE rounds of quantizer lanes) and the first LPRE la partial
  //    slots of this thread's la value
  constexpr int QPRE = 2, LPRE = 32;
  const int lanes_per_row = K / 8, qlanes = M * lanes_per_row;
  v4i xpre[QPRE], spre[QPRE];
#pragma unroll
  for (int q = 0; q < QPRE; ++q) {
    const int li = q * GV_THREADS + tid;
    xpre[q] = spre[q] = (v4i){0, 0, 0, 0};
    if (li < qlanes) {
      const int m = li / lanes_per_row, e8 = li - m * lanes_per_row;
      xpre[q] = *(const v4i*)(x + (int64_t)m * ldx + 8 * e8);
      if (smooth) spre[q] = *(const v4i*)(smooth + 8 * e8);
    }
  }
  float lpre[LPRE];
  const int64_t MR = (int64_t)M * R;
  if constexpr (RB > 0) {
#pragma unroll
    for (int p = 0; p < LPRE; ++p) lpre[p] = (tid < MR && p < P) ? la_part[p * MR + tid] : 0.0f;
  }
  const float s2 = s2p ? *s2p : 1.0f;

  // 1. this workgroup's weight bytes and scales (the stream; first needed in step 3)
  v4i wv[GV_MAX_ITEMS][2];
  // the scales as 32-bit values: each load gets a register of its own (held as 16-bit values, they went
  // through one temporary register, and every item's loads waited for the previous item's scale)
  uint32_t swv[GV_MAX_ITEMS];
  // Branch-free: an item index past the workgroup's items re-reads its last item (one broadcast line, never
  // used), so every load goes out in one batch with nothing to merge.
#pragma unroll
  for (int it = 0; it < GV_MAX_ITEMS; ++it) {
    const int item = min(it * GV_THREADS + tid, items - 1);
    const int r = item / G, g = item - r * G;
    const uint8_t* wp = qw + (int64_t)(n0 + r) * (K / 2) + g * 32;
    wv[it][0] = *(const v4i*)wp;
    wv[it][1] = *(const v4i*)(wp + 16);
    swv[it] = sw[(int64_t)(n0 + r) * G + g];
  }

  // 2. activation codes and scales (kernel 1's quantizer; a group = 8 consecutive lanes, 8 elements each)
  const bool s2_one = s2 == 1.0f;
  for (int base = 0, q = 0; base < qlanes; base += GV_THREADS, ++q) {  // uniform trip count: quant8 is wave-collective
    const int li = base + tid;
    const bool valid = li < qlanes;
    const int m = valid ? li / lanes_per_row : 0, e8 = valid ? li - m * lanes_per_row : 0;
    v4i c = (v4i){0, 0, 0, 0}, sv = (v4i){0, 0, 0, 0};
    if (q < QPRE) {
#pragma unroll
      for (int u = 0; u < QPRE; ++u)
        if (u == q) c = xpre[u], sv = spre[u];
    } else if (valid) {
      c = *(const v4i*)(x + (int64_t)m * ldx + 8 * e8);
      if (smooth) sv = *(const v4i*)(smooth + 8 * e8);
    }
    uint32_t w[4];
    if (smooth && valid) {
      float f[8];
      bool ok = true;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f[2 * t] = bf16_lo((uint32_t)sv[t]);
        f[2 * t + 1] = bf16_hi((uint32_t)sv[t]);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) ok = ok && g64::smooth_ok(f[t]);
      if (ok) {
#pragma unroll
        for (int t = 0; t < 8; ++t) f[t] = 1.0f / f[t];
      }
      g64::smooth8(c, f, !ok, w);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) w[t] = (uint32_t)c[t];
    }
    uint32_t nb[2];
    uint16_t sh;
    g64::quant8(w, valid, s2_one, s2, nb, sh);
    if (valid) {
      codes[(m * G + (e8 >> 3)) * L.cs + (e8 & 7)] = pack_nibbles8(nb);
      if ((e8 & 7) == 0) sxl[m * G + (e8 >> 3)] = f16_bits_to_f32(sh);
    }
  }
  // la = RN_bf16(sum of the partial slots in slot order)
  if constexpr (RB > 0) {
    for (int64_t i = tid; i < MR; i += GV_THREADS) {
      float s;
      if (i == tid) {
        s = lpre[0];
#pragma unroll
        for (int p = 1; p < LPRE; ++p)
          if (p < P) s += lpre[p];
        for (int p = LPRE; p < P; ++p) s += la_part[p * MR + i];
      } else {
        s = la_part[i];
        for (int p = 1; p < P; ++p) s += la_part[p * MR + i];
      }
      lal[i] = bf16_to_f32(f32_to_bf16(s));
    }
  }
  __syncthreads();

  // 3. exact group dot products
#pragma unroll
  for (int it = 0; it < GV_MAX_ITEMS; ++it) {
    const int item = it * GV_THREADS + tid;
    if (item < items) {
      const int r = item / G, g = item - r * G;
      swl[r * L.gp + g] = f16_bits_to_f32((uint16_t)swv[it]);
      for (int m = 0; m < M; ++m) {
        const uint32_t* a = codes + (m * G + g) * L.cs;
        int d = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          d = __builtin_amdgcn_sdot8((int)a[j], wv[it][0][j], d, false);
          d = __builtin_amdgcn_sdot8((int)a[4 + j], wv[it][1][j], d, false);
        }
        pl[(m * GV_ROWS + r) * L.gp + g] = (float)d;
      }
    }
  }
  __syncthreads();

  // 4. per (token, row): the group chain in the GEMM's order, then the epilogue
  if (tid < M * GV_ROWS) {
    const int m = tid / GV_ROWS, r = tid - m * GV_ROWS, n = n0 + r;
    const float* pp = pl + (m * GV_ROWS + r) * L.gp;
    const float* sxm = sxl + m * G;
    const float* swr = swl + r * L.gp;
    float acc = 0.0f;
#pragma unroll 8
    for (int g = 0; g < G; ++g) acc = __builtin_fmaf(pp[g], sxm[g] * swr[g], acc);  // LDS reads batched by 8
    float mult = s2;
    if (second) mult *= second[second_per_channel ? n : 0];
    float y;
    if constexpr (RB > 0) {
      y = acc * mult;
      const uint16_t* ur = up + (int64_t)n * R;
#pragma unroll 4
      for (int k = 0; k < R; k += 8) {
        const v4i u = *(const v4i*)(ur + k);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          y = __builtin_fmaf(lal[m * R + k + 2 * e], bf16_lo((uint32_t)u[e]), y);
          y = __builtin_fmaf(lal[m * R + k + 2 * e + 1], bf16_hi((uint32_t)u[e]), y);
        }
      }
      if (bias) y += bf16_to_f32(bias[n]);
    } else {
      // without a low-rank term the GEMM's epilogue forms acc * mult + bias as one fma
      y = bias ? __builtin_fmaf(acc, mult, bf16_to_f32(bias[n])) : acc * mult;
    }
    if (gelu) y = gelu_tanh_f32(y);
    out[(int64_t)m * N + n] = out_f16 ? f32_to_f16_bits(y) : f32_to_bf16(y);
  }
}

// activation records (+ 1 KB slack) and la partial slots of kernel 1, 256-byte aligned pieces
int64_t records_bytes(int64_t M, int64_t K) { return ((K / 128) * M * GWA_FP6_REC + 1024 + 255) / 256 * 256; }

}  // namespace

extern "C" int gwa_svdq_w4a4_gemv_max_m(int64_t K, int64_t rank) {
  if (K <= 0 || K % 128 || K > 64 * GV_MAX_ITEMS * GV_THREADS / 16) return 0;
  if (!(rank == 0 || rank == 16 || rank == 32 || rank == 64 || rank == 128)) return 0;
  int m = GV_MAX_M;
  while (m > 0 && gv_budget_bytes((int)m, (int)K, (int)rank, 16) > 64 * 1024) --m;
  return m;
}

extern "C" int64_t gwa_svdq_w4a4_linear_gemv_workspace(int64_t M, int64_t K, int64_t rank) {
  if (M <= 0 || K <= 0 || K % 128 || rank < 0) return 0;
  if (rank == 0) return 256;
  return records_bytes(M, K) + gwa_svdq_quant_fp6_la_workspace(M, K, rank);
}

extern "C" int gwa_svdq_w4a4_linear_gemv(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                         const void* proj_down_op6, int64_t rank, const uint8_t* qw, const void* sw,
                                         const float* second, int64_t second_numel, const void* proj_up,
                                         const void* bias, void* out, int out_dtype, int epilogue_flags, int64_t M,
                                         int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                                         void* stream) {
  const char* what = "svdq_w4a4_linear_gemv";
  GWA_REQUIRE(K > 0 && K % 128 == 0, "%s: K=%lld is not a multiple of 128", what, (long long)K);
  GWA_REQUIRE(N > 0 && N % 16 == 0 && N < (1ll << 31), "%s: N=%lld is not a positive multiple of 16", what,
              (long long)N);
  GWA_REQUIRE((proj_down_op6 == nullptr) == (proj_up == nullptr),
              "%s: proj_down_op6 and proj_up must both be given or both be NULL", what);
  const int64_t R = proj_up ? rank : 0;
  const int max_m = gwa_svdq_w4a4_gemv_max_m(K, R);
  GWA_REQUIRE(max_m > 0, "%s: K=%lld rank=%lld is not served by the small-M path", what, (long long)K,
              (long long)R);
  GWA_REQUIRE(M >= 0 && M <= max_m, "%s: M=%lld above the small-M path's %d tokens at K=%lld", what, (long long)M,
              max_m, (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "%s: row stride %lld must be >= K and a multiple of 8", what,
              (long long)ldx);
  GWA_REQUIRE(out_dtype == GWA_DT_BF16 || out_dtype == GWA_DT_F16, "%s: out_dtype %d", what, out_dtype);
  GWA_REQUIRE((epilogue_flags & ~GWA_EPI_GELU_TANH) == 0, "%s: unknown epilogue flags 0x%x", what, epilogue_flags);
  GWA_REQUIRE(second == nullptr || second_numel == 1 || second_numel == N, "%s: second has %lld values for N=%lld",
              what, (long long)second_numel, (long long)N);
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && qw && sw && out, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(qw, 16) && GWA_ALIGNED(sw, 2) && GWA_ALIGNED(smooth, 16) &&
                  GWA_ALIGNED(proj_up, 16) && GWA_ALIGNED(out, 2) && GWA_ALIGNED(bias, 2) && GWA_ALIGNED(second, 4) &&
                  GWA_ALIGNED(s2, 4) && GWA_ALIGNED(workspace, 256),
              "%s: x, qw, smooth and proj_up must be 16-byte aligned, workspace 256-byte", what);
  const int64_t need = gwa_svdq_w4a4_linear_gemv_workspace(M, K, R);
  GWA_REQUIRE(workspace && workspace_bytes >= need, "%s: workspace of %lld bytes, %lld needed", what,
              (long long)workspace_bytes, (long long)need);
  hipStream_t st = (hipStream_t)stream;
  const float* la_part = nullptr;
  int P = 0;
  if (R > 0) {
    // kernel 1 for la's partial slots (its records are not read: this path quantizes the rows itself)
    uint8_t* ws = (uint8_t*)workspace;
    float* part = (float*)(ws + records_bytes(M, K));
    const int rc = gwa_svdq_quant_fp6(x, ldx, smooth, s2, proj_down_op6, R, ws, part, M, K, stream);
    if (rc != GWA_OK) return rc;
    la_part = part;
    P = (int)gwa_svdq_quant_fp6_partials(M, K, R);
  }
  // 32 rows per workgroup (half the workgroups: one round over the CUs at the modulation shapes) where the
  // items and LDS allow, else 16
  const int G = (int)(K / 64);
  const bool rows32 = G * 32 <= GV_MAX_ITEMS * GV_THREADS && N % 32 == 0 &&
                      gv_budget_bytes((int)M, (int)K, (int)R, 32) <= 64 * 1024;
  const int rows = rows32 ? 32 : 16;
  const GvLds L((int)M, (int)K, (int)R, rows);
  const dim3 grid((unsigned)(N / rows)), block(GV_THREADS);
  const int sec_pc = second_numel > 1 ? 1 : 0, gelu = (epilogue_flags & GWA_EPI_GELU_TANH) ? 1 : 0,
            f16 = out_dtype == GWA_DT_F16 ? 1 : 0;
  const uint16_t *xp = (const uint16_t*)x, *smp = (const uint16_t*)smooth, *swp = (const uint16_t*)sw,
                 *upp = (const uint16_t*)proj_up, *bp = (const uint16_t*)bias;
  uint16_t* op = (uint16_t*)out;
  const int m = (int)M, n = (int)N, k = (int)K;
#define GWA_GV_LAUNCH(RBV)                                                                                        \
  if (rows32)                                                                                                     \
    hipLaunchKernelGGL((svdq_gemv_w4a4_kernel<RBV, 32>), grid, block, (unsigned)L.total, st, xp, ldx, smp, s2,  \
                       la_part, P, qw, swp, second, sec_pc, upp, bp, op, gelu, f16, m, n, k);                     \
  else                                                                                                            \
    hipLaunchKernelGGL((svdq_gemv_w4a4_kernel<RBV, 16>), grid, block, (unsigned)L.total, st, xp, ldx, smp, s2,  \
                       la_part, P, qw, swp, second, sec_pc, upp, bp, op, gelu, f16, m, n, k)
  switch (R / 16) {
    case 0: GWA_GV_LAUNCH(0); break;
    case 1: GWA_GV_LAUNCH(1); break;
    case 2: GWA_GV_LAUNCH(2); break;
    case 4: GWA_GV_LAUNCH(4); break;
    case 8: GWA_GV_LAUNCH(8); break;
    default: return gwa_set_error(GWA_ERR_INVALID, "%s: rank %lld", what, (long long)R);
  }
#undef GWA_GV_LAUNCH
  return gwa_check_launch(what);
}
