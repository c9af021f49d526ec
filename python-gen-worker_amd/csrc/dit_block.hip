// Block glue of the Flux-shaped DiT that the benchmark's denoiser step runs: the ops between the linears of
// diffusers' FluxTransformerBlock / FluxSingleTransformerBlock, fused into one pass each so that the step is
// dominated by the linears and attention, as it is in the reference's serving path, and not by chains of
// small elementwise launches. The model calls them in both of its lanes (W4A4 and bf16 linears).
//
//  * qk norm + rotary: per token and head, q and k -> RMSNorm over head_dim (fp32 sum of squares, rsqrt of
//    mean + eps, bf16 rounding, times the bf16 weight) -> rotary embedding on interleaved (even, odd) pairs,
//    every product and sum rounded to bf16 as the torch expression rounds it; v copied alongside, so the
//    outputs can be rows of the joint [text; image] sequence without a concatenation.
//  * adaLN modulate: LayerNorm without affine (fp32 mean and variance, rsqrt(var + eps)) rounded to bf16,
//    times bf16(1 + scale), plus shift, each step rounded to bf16.
//  * gated residual: x + bf16(gate * y), gate broadcast over rows.
//
// The roundings follow the torch expressions the model states them with (flux_dit.py); only the order of
// the fp32 sums inside a row's mean and variance differs from torch's reduction kernels.
#include "gwa_common.h"

namespace {

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// butterfly sum over the 64 lanes: every lane ends with the same value, in a fixed order
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ---------------------------------------------------------------------------------------------------------
// qk norm + rotary (+ v copy). One wave per (token, head); head_dim 128, lane l holds pair (2l, 2l + 1).
// ---------------------------------------------------------------------------------------------------------
constexpr int QK_WAVES = 4;

__device__ __forceinline__ uint32_t norm_rope_pair(uint32_t u, uint32_t w, float c, float s, float eps) {
  const float e = bf16_lo(u), o = bf16_hi(u);
  const float ss = wave_sum(e * e + o * o);
  const float r = rsqrtf(ss * (1.0f / 128.0f) + eps);
  const float ye = bf16r(bf16r(e * r) * bf16_lo(w));
  const float yo = bf16r(bf16r(o * r) * bf16_hi(w));
  const float oe = bf16r(bf16r(ye * c) - bf16r(yo * s));
  const float oo = bf16r(bf16r(ye * s) + bf16r(yo * c));
  return (uint32_t)f32_to_bf16(oe) | ((uint32_t)f32_to_bf16(oo) << 16);
}

__global__ __launch_bounds__(64 * QK_WAVES) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ xq, const uint16_t* __restrict__ xk, const uint16_t* __restrict__ xv, int64_t ldx,
    const uint16_t* __restrict__ wq, const uint16_t* __restrict__ wk, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int64_t pos0, uint16_t* __restrict__ oq, uint16_t* __restrict__ ok,
    uint16_t* __restrict__ ov, int64_t ldo, int64_t items, int heads, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * QK_WAVES + (threadIdx.x >> 6);
  if (item >= items) return;  // wave-uniform
  const int64_t row = item / heads;
  const int h = (int)(item - row * heads);
  const int64_t xi = row * ldx + h * 128 + 2 * lane, oi = row * ldo + h * 128 + 2 * lane;
  const int64_t ti = (pos0 + row) * 64 + lane;
  const uint32_t uq = *(const uint32_t*)(xq + xi), uk = *(const uint32_t*)(xk + xi);
  const uint32_t uv = xv ? *(const uint32_t*)(xv + xi) : 0u;
  const float c = bf16_to_f32(cos_t[ti]), s = bf16_to_f32(sin_t[ti]);
  const uint32_t gq = *(const uint32_t*)(wq + 2 * lane), gk = *(const uint32_t*)(wk + 2 * lane);
  *(uint32_t*)(oq + oi) = norm_rope_pair(uq, gq, c, s, eps);
  *(uint32_t*)(ok + oi) = norm_rope_pair(uk, gk, c, s, eps);
  if (xv) *(uint32_t*)(ov + oi) = uv;
}

// Wide form (16-byte aligned rows): one wave per token and 4 heads, 16 lanes per head, lane holding 8
// consecutive values (4 rotary pairs); the sum of squares is the lane's 4 pair sums, then a butterfly over the
// head's 16 lanes. 16-byte loads and stores, a quarter of the waves and shuffles of the form above.
__device__ __forceinline__ float head_sum16(float v) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ v4i norm_rope8(v4i u, v4i w, uint2 cs, uint2 sn, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float e = bf16_lo((uint32_t)u[i]), o = bf16_hi((uint32_t)u[i]);
    ss += e * e + o * o;
  }
  const float r = rsqrtf(head_sum16(ss) * (1.0f / 128.0f) + eps);
  v4i out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float e = bf16_lo((uint32_t)u[i]), o = bf16_hi((uint32_t)u[i]);
    const uint32_t cw = i < 2 ? cs.x : cs.y, sw = i < 2 ? sn.x : sn.y;
    const float c = (i & 1) ? bf16_hi(cw) : bf16_lo(cw), s = (i & 1) ? bf16_hi(sw) : bf16_lo(sw);
    const float ye = bf16r(bf16r(e * r) * bf16_lo((uint32_t)w[i]));
    const float yo = bf16r(bf16r(o * r) * bf16_hi((uint32_t)w[i]));
    const float oe = bf16r(bf16r(ye * c) - bf16r(yo * s));
    const float oo = bf16r(bf16r(ye * s) + bf16r(yo * c));
    out[i] = (int)((uint32_t)f32_to_bf16(oe) | ((uint32_t)f32_to_bf16(oo) << 16));
  }
  return out;
}

__global__ __launch_bounds__(64 * QK_WAVES) void qk_norm_rope_wide_kernel(
    const uint16_t* __restrict__ xq, const uint16_t* __restrict__ xk, const uint16_t* __restrict__ xv, int64_t ldx,
    const uint16_t* __restrict__ wq, const uint16_t* __restrict__ wk, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int64_t pos0, uint16_t* __restrict__ oq, uint16_t* __restrict__ ok,
    uint16_t* __restrict__ ov, int64_t ldo, int64_t items, int heads, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * QK_WAVES + (threadIdx.x >> 6);
  if (item >= items) return;  // wave-uniform
  const int hgroups = (heads + 3) >> 2;
  const int64_t row = item / hgroups;
  const int h = (int)(item - row * hgroups) * 4 + (lane >> 4), e8 = 8 * (lane & 15);
  if (h >= heads) return;  // a whole 16-lane group: its butterfly stays inside the group
  const int64_t xi = row * ldx + h * 128 + e8, oi = row * ldo + h * 128 + e8;
  const int64_t ti = (pos0 + row) * 64 + (e8 >> 1);
  const v4i uq = *(const v4i*)(xq + xi), uk = *(const v4i*)(xk + xi);
  const uint2 cs = *(const uint2*)(cos_t + ti), sn = *(const uint2*)(sin_t + ti);
  const v4i gq = *(const v4i*)(wq + e8), gk = *(const v4i*)(wk + e8);
  if (xv) *(v4i*)(ov + oi) = *(const v4i*)(xv + xi);
  *(v4i*)(oq + oi) = norm_rope8(uq, gq, cs, sn, eps);
  *(v4i*)(ok + oi) = norm_rope8(uk, gk, cs, sn, eps);
}

// ---------------------------------------------------------------------------------------------------------
// adaLN modulate (see the kernel's comment for the split of a row over waves).
// ---------------------------------------------------------------------------------------------------------
constexpr int LN_RPB = 2;  // rows per workgroup

// adaLN modulate: WPR waves share a row of C = 512 * NCH columns (NCH / WPR 512-column chunks each, lane l
// holding columns 512 j + 8 l .. + 8; their partial sums are added in wave order through LDS), LN_RPB rows
// per workgroup
template <int NCH, int WPR>
__global__ __launch_bounds__(64 * WPR * LN_RPB) void adaln_modulate_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ shift, uint16_t* __restrict__ out, int64_t ldo, int64_t rows, float eps) {
  constexpr int C = 512 * NCH, NJ = NCH / WPR;
  static_assert(NCH % WPR == 0, "chunks per wave");
  __shared__ float red[WPR * LN_RPB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wr = wave / WPR, wq = wave - wr * WPR;
  const int64_t row = (int64_t)blockIdx.x * LN_RPB + wr;
  const int j0 = wq * NJ;
  const bool ok = row < rows;
  float v[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const v4i u = ok ? *(const v4i*)(x + row * ldx + 512 * (j0 + j) + 8 * lane) : (v4i){0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[j][2 * e] = bf16_lo((uint32_t)u[e]);
      v[j][2 * e + 1] = bf16_hi((uint32_t)u[e]);
    }
  }
  auto row_sum = [&](float t) __attribute__((always_inline)) {  // the row's total, its waves' parts in order
    t = wave_sum(t);
    if constexpr (WPR > 1) {
      if (lane == 0) red[wave] = t;
      __syncthreads();
      t = red[wr * WPR];
#pragma unroll
      for (int i = 1; i < WPR; ++i) t += red[wr * WPR + i];
      __syncthreads();
    }
    return t;
  };
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += v[j][e];
  const float mean = row_sum(sum) / (float)C;
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = v[j][e] - mean;
      sq = __builtin_fmaf(d, d, sq);
    }
  const float rstd = rsqrtf(row_sum(sq) / (float)C + eps);
  if (!ok) return;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int col = 512 * (j0 + j) + 8 * lane;
    const v4i us = *(const v4i*)(scale + col), uh = *(const v4i*)(shift + col);
    v4i o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r2[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const float sc = b ? bf16_hi((uint32_t)us[e]) : bf16_lo((uint32_t)us[e]);
        const float sh = b ? bf16_hi((uint32_t)uh[e]) : bf16_lo((uint32_t)uh[e]);
        const float y = bf16r((v[j][2 * e + b] - mean) * rstd);
        r2[b] = bf16r(bf16r(y * bf16r(1.0f + sc)) + sh);
      }
      o[e] = (int)((uint32_t)f32_to_bf16(r2[0]) | ((uint32_t)f32_to_bf16(r2[1]) << 16));
    }
    *(v4i*)(out + row * ldo + col) = o;
  }
}

// ---------------------------------------------------------------------------------------------------------
// gated residual: out = x + bf16(gate * y). One thread per 8 columns.
// ---------------------------------------------------------------------------------------------------------
// out may be x (in place): each thread reads its 8 columns of x before it writes them
__global__ __launch_bounds__(256) void gate_residual_kernel(const uint16_t* x, int64_t ldx,
                                                            const uint16_t* __restrict__ y, int64_t ldy,
                                                            const uint16_t* __restrict__ gate,
                                                            uint16_t* out, int64_t ldo, int64_t rows, int C) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int per_row = C / 8;
  const int64_t row = t / per_row;
  if (row >= rows) return;
  const int col = (int)(t - row * per_row) * 8;
  const v4i ux = *(const v4i*)(x + row * ldx + col), uy = *(const v4i*)(y + row * ldy + col);
  const v4i ug = *(const v4i*)(gate + col);
  v4i o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t a = (uint32_t)ux[e], b = (uint32_t)uy[e], g = (uint32_t)ug[e];
    const float lo = bf16r(bf16_lo(a) + bf16r(bf16_lo(g) * bf16_lo(b)));
    const float hi = bf16r(bf16_hi(a) + bf16r(bf16_hi(g) * bf16_hi(b)));
    o[e] = (int)((uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16));
  }
  *(v4i*)(out + row * ldo + col) = o;
}

}  // namespace

extern "C" int gwa_dit_qk_norm_rope(const void* xq, const void* xk, const void* xv, int64_t ldx, const void* wq,
                                    const void* wk, const void* cos_t, const void* sin_t, int64_t pos0,
                                    int64_t table_rows, void* oq, void* ok, void* ov, int64_t ldo, int64_t rows,
                                    int64_t heads, int64_t head_dim, float eps, void* stream) {
  const char* what = "dit_qk_norm_rope";
  GWA_REQUIRE(head_dim == 128, "%s: head_dim %lld (only 128 is built)", what, (long long)head_dim);
  GWA_REQUIRE(rows >= 0 && heads > 0 && heads <= 4096, "%s: bad shape rows=%lld heads=%lld", what,
              (long long)rows, (long long)heads);
  GWA_REQUIRE(ldx >= heads * head_dim && ldo >= heads * head_dim && ldx % 2 == 0 && ldo % 2 == 0,
              "%s: row strides ldx=%lld ldo=%lld must be even and >= heads * head_dim", what, (long long)ldx,
              (long long)ldo);
  GWA_REQUIRE(pos0 >= 0 && pos0 + rows <= table_rows, "%s: positions [%lld, %lld) outside the %lld-row tables",
              what, (long long)pos0, (long long)(pos0 + rows), (long long)table_rows);
  GWA_REQUIRE((xv == nullptr) == (ov == nullptr), "%s: xv and ov must both be given or both be NULL", what);
  if (rows == 0) return GWA_OK;
  GWA_REQUIRE(xq && xk && wq && wk && cos_t && sin_t && oq && ok, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(xq, 4) && GWA_ALIGNED(xk, 4) && GWA_ALIGNED(xv, 4) && GWA_ALIGNED(wq, 4) &&
                  GWA_ALIGNED(wk, 4) && GWA_ALIGNED(oq, 4) && GWA_ALIGNED(ok, 4) && GWA_ALIGNED(ov, 4),
              "%s: tensors must be 4-byte aligned", what);
  const bool wide = GWA_ALIGNED(xq, 16) && GWA_ALIGNED(xk, 16) && GWA_ALIGNED(xv, 16) && GWA_ALIGNED(wq, 16) &&
                    GWA_ALIGNED(wk, 16) && GWA_ALIGNED(oq, 16) && GWA_ALIGNED(ok, 16) && GWA_ALIGNED(ov, 16) &&
                    GWA_ALIGNED(cos_t, 8) && GWA_ALIGNED(sin_t, 8) && ldx % 8 == 0 && ldo % 8 == 0;
  const int64_t items = rows * (wide ? (heads + 3) / 4 : heads);
  const int64_t blocks = (items + QK_WAVES - 1) / QK_WAVES;
  GWA_REQUIRE(blocks < (1ll << 31), "%s: grid too large", what);
  hipLaunchKernelGGL(wide ? qk_norm_rope_wide_kernel : qk_norm_rope_kernel, dim3((unsigned)blocks),
                     dim3(64 * QK_WAVES), 0, (hipStream_t)stream,
                     (const uint16_t*)xq, (const uint16_t*)xk, (const uint16_t*)xv, ldx, (const uint16_t*)wq,
                     (const uint16_t*)wk, (const uint16_t*)cos_t, (const uint16_t*)sin_t, pos0, (uint16_t*)oq,
                     (uint16_t*)ok, (uint16_t*)ov, ldo, items, (int)heads, eps);
  return gwa_check_launch(what);
}

extern "C" int gwa_dit_adaln_modulate(const void* x, int64_t ldx, const void* scale, const void* shift, void* out,
                                      int64_t ldo, int64_t rows, int64_t cols, float eps, void* stream) {
  const char* what = "dit_adaln_modulate";
  GWA_REQUIRE(cols > 0 && cols % 512 == 0 && cols <= 4096, "%s: cols=%lld must be a multiple of 512, <= 4096",
              what, (long long)cols);
  GWA_REQUIRE(rows >= 0 && ldx >= cols && ldo >= cols && ldx % 8 == 0 && ldo % 8 == 0,
              "%s: row strides ldx=%lld ldo=%lld must be multiples of 8 and >= cols", what, (long long)ldx,
              (long long)ldo);
  if (rows == 0) return GWA_OK;
  GWA_REQUIRE(x && scale && shift && out, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(scale, 16) && GWA_ALIGNED(shift, 16) && GWA_ALIGNED(out, 16),
              "%s: tensors must be 16-byte aligned", what);
  const int64_t blocks = (rows + LN_RPB - 1) / LN_RPB;
  GWA_REQUIRE(blocks < (1ll << 31), "%s: grid too large", what);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *xp = (const uint16_t*)x, *sc = (const uint16_t*)scale, *sh = (const uint16_t*)shift;
  uint16_t* op = (uint16_t*)out;
  // two waves per row where the chunks split evenly (3072 columns: 23.3 -> 21.5 us at 4608 rows against one
  // wave per row; three or six waves per row: 22.1 and 23.1 us), else one
#define GWA_LN_CASE(N, W)                                                                                        \
  case N:                                                                                                        \
    hipLaunchKernelGGL((adaln_modulate_kernel<N, W>), dim3((unsigned)blocks), dim3(64 * W * LN_RPB), 0, st, xp, ldx, \
                       sc, sh, op, ldo, rows, eps);                                                              \
    break;
  switch (cols / 512) {
    GWA_LN_CASE(1, 1) GWA_LN_CASE(2, 2) GWA_LN_CASE(3, 1) GWA_LN_CASE(4, 2) GWA_LN_CASE(5, 1) GWA_LN_CASE(6, 2)
    GWA_LN_CASE(7, 1) GWA_LN_CASE(8, 2)
    default: return gwa_set_error(GWA_ERR_INVALID, "%s: cols=%lld", what, (long long)cols);
  }
#undef GWA_LN_CASE
  return gwa_check_launch(what);
}

extern "C" int gwa_dit_gate_residual(const void* x, int64_t ldx, const void* y, int64_t ldy, const void* gate,
                                     void* out, int64_t ldo, int64_t rows, int64_t cols, void* stream) {
  const char* what = "dit_gate_residual";
  GWA_REQUIRE(cols > 0 && cols % 8 == 0 && cols < (1ll << 24), "%s: cols=%lld must be a positive multiple of 8",
              what, (long long)cols);
  GWA_REQUIRE(rows >= 0 && ldx >= cols && ldy >= cols && ldo >= cols && ldx % 8 == 0 && ldy % 8 == 0 &&
                  ldo % 8 == 0,
              "%s: row strides must be multiples of 8 and >= cols", what);
  if (rows == 0) return GWA_OK;
  GWA_REQUIRE(x && y && gate && out, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(y, 16) && GWA_ALIGNED(gate, 16) && GWA_ALIGNED(out, 16),
              "%s: tensors must be 16-byte aligned", what);
  const int64_t threads = rows * (cols / 8), blocks = (threads + 255) / 256;
  GWA_REQUIRE(blocks < (1ll << 31), "%s: grid too large", what);
  hipLaunchKernelGGL(gate_residual_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, ldx, (const uint16_t*)y, ldy, (const uint16_t*)gate, (uint16_t*)out, ldo,
                     rows, (int)cols);
  return gwa_check_launch(what);
}
