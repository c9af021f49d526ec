// Attention of the benchmark's Flux-shaped DiT (joint [text; image] self-attention, no mask, head_dim 128,
// bf16 in and out): softmax(q k^T / sqrt(128)) v per head in one pass over the keys with an online softmax
// (the flash-attention recurrence), in place of torch's scaled_dot_product_attention (which diffusers'
// FluxAttnProcessor calls; here the vendor kernel ran at ~0.49 PFLOP/s).
//
// Work split: a 512-thread workgroup owns 256 queries of one head (8 waves x 32 queries) and walks the keys
// in tiles of 128. K and V tiles ([128 keys][128], as stored) are copied global -> LDS by direct-to-LDS
// buffer loads (no staging registers, no LDS writes), double buffered: tile t+1's copies are issued before
// tile t's MFMAs, one wait and one barrier per tile. The 16-byte chunks of a row are XOR-swizzled by the
// row at copy time (each lane fetches the chunk that belongs at its LDS slot), so the reads below are free
// of bank conflicts. Each wave computes, with bf16 MFMA 32x32x16 and fp32 accumulation:
//   S^T = K_tile q^T            (keys x queries: a lane holds one query and 16 keys of each 32-key half)
//   p   = exp2(S * c - m)       (c = log2(e) / sqrt(128), m the query's running max: the two lane halves
//                                exchange their maxima; O is rescaled only in tiles where some lane's max
//                                moved; the row sums stay per lane until the end)
//   O^T = O^T * exp2(m_old - m) + V^T p^T   (head_dim x queries: a lane holds one query's 64 outputs)
// The V^T operand comes straight from the row-major V tile through ds_read_b64_tr_b16: in each 16-lane group
// lane i receives element e of the 8-byte read of lane 4e + i/4, column i % 4, so lanes that point at 4 keys
// x 16 head-dim columns hand each lane 4 keys of one column. The key order inside a 16-key MFMA step is the
// one S^T's output layout leaves p in, so p goes from the S MFMA to the O MFMA without leaving registers.
// Output o = O / l in bf16, written as rows [query][head][128] (the layout the next linear reads).
#include <type_traits>

#include "fp6_gemm_common.h"

namespace {

// 8 waves per workgroup (one workgroup per CU): each K / V tile copy serves 256 queries (4 waves: 128, two
// workgroups per CU, 319 -> 303 us at 4608 tokens x 24 heads); 128-key tiles halve the waits and barriers
// per key (64-key tiles: 303 -> 298 us)
constexpr int AT_D = 128, AT_BN = 128, AT_NW = 8, AT_BM = 32 * AT_NW, AT_THREADS = 64 * AT_NW;
constexpr int AT_NSB = AT_BN / 32, AT_NC = AT_BN / 16;  // 32-key halves and 16-key MFMA steps of a tile
constexpr int AT_RUNS = AT_BN / 4 / AT_NW;  // 1 KB copy runs (4 rows) per wave, per K and per V tile
constexpr int AT_ROW = AT_D * 2;                       // tile row bytes (256), chunks swizzled, no padding
constexpr int AT_TILE = AT_BN * AT_ROW;                // 32 KB per K or V tile
constexpr int AT_STAGE = 2 * AT_TILE;                  // K then V
constexpr int AT_LDS = 2 * AT_STAGE;                   // 128 KB

typedef float v16f_ __attribute__((ext_vector_type(16)));
typedef short v4s_ __attribute__((ext_vector_type(4)));
typedef short v2s_ __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16_pair(float a, float b) { return pack_bf16x2_rn(a, b); }

// 16-byte chunk slot of chunk ch in tile row r: K rows XOR the row's low 4 bits (16-byte reads by 16 rows
// hit distinct banks), V rows XOR an even value (the two chunks of a 32-byte run stay adjacent for the
// transposing 8-byte reads, which take 4 rows x 32 bytes per 16-lane group)
__device__ __forceinline__ int k_slot(int ch, int r) { return ch ^ (r & 15); }
__device__ __forceinline__ int v_slot(int ch, int r) { return ch ^ (2 * (r & 7)); }

__device__ __forceinline__ v4s_ lds_read_tr(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_*)(uintptr_t)p);
}

__global__ __launch_bounds__(AT_THREADS, 8 / AT_NW) void dit_attention_kernel(
    const uint16_t* __restrict__ q, int64_t ldq, const uint16_t* __restrict__ k, int64_t ldk,
    const uint16_t* __restrict__ v, int64_t ldv, uint16_t* __restrict__ o, int64_t ldo, int S, int Skv,
    float c_log2) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[AT_LDS];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int j = lane & 31, h = lane >> 5;              // MFMA column (query / key / head-dim row) and half
  const int head = blockIdx.y;
  const int q0 = blockIdx.x * AT_BM + wave * 32;
  const int qrow = q0 + j;
  const bool q_ok = qrow < S;

  // q^T operand (B of the S MFMA): lane (j, h) holds q[qrow][16 cd + 8 h .. + 8] for cd = 0..7
  v4i qop[8];
  {
    const uint16_t* qp = q + (int64_t)(q_ok ? qrow : 0) * ldq + head * AT_D + 8 * h;
#pragma unroll
    for (int cd = 0; cd < 8; ++cd) qop[cd] = q_ok ? *(const v4i*)(qp + 16 * cd) : (v4i){0, 0, 0, 0};
  }

  // copies: 32 runs of 1 KB (4 rows) per K tile and per V tile, runs wave + 8 u of each; lane l of a
  // run lands at LDS slot l % 16 of row 4 run + l / 16 and fetches the chunk that belongs there
  const v4i kbuf = raw_rsrc(k, (uint32_t)(((int64_t)(Skv - 1) * ldk + gridDim.y * AT_D) * 2));
  const v4i vbuf = raw_rsrc(v, (uint32_t)(((int64_t)(Skv - 1) * ldv + gridDim.y * AT_D) * 2));
  uint32_t koff[AT_RUNS], voff[AT_RUNS];
#pragma unroll
  for (int u = 0; u < AT_RUNS; ++u) {
    const int run = wave + AT_NW * u, row = 4 * run + (lane >> 4), slot = lane & 15;
    koff[u] = (uint32_t)((row * ldk + head * AT_D + 8 * k_slot(slot, row)) * 2);
    voff[u] = (uint32_t)((row * ldv + head * AT_D + 8 * v_slot(slot, row)) * 2);
  }
  // tile t into stage buffer b; a last tile with rv < 128 keys repeats its last key in the rows past it (their
  // scores are masked to -inf below, so they weigh 0)
  auto issue = [&](int t, int b, int rv) __attribute__((always_inline)) {
    uint8_t* kb = lds + b * AT_STAGE;
    const uint32_t ks = (uint32_t)((int64_t)t * AT_BN * ldk * 2), vs = (uint32_t)((int64_t)t * AT_BN * ldv * 2);
#pragma unroll
    for (int u = 0; u < AT_RUNS; ++u) {
      const int run = wave + AT_NW * u;
      uint32_t ko = koff[u], vo = voff[u];
      if (rv < AT_BN) {  // workgroup-uniform: the last, partial tile
        const int row = 4 * run + (lane >> 4), slot = lane & 15, src = min(row, rv - 1);
        ko = (uint32_t)((src * ldk + head * AT_D + 8 * k_slot(slot, row)) * 2);
        vo = (uint32_t)((src * ldv + head * AT_D + 8 * v_slot(slot, row)) * 2);
      }
      dma16(kbuf, (uint32_t)(uintptr_t)(kb + run * 1024), ko, ks);
      dma16(vbuf, (uint32_t)(uintptr_t)(kb + AT_TILE + run * 1024), vo, vs);
    }
  };

  // read offsets, loop-invariant: K rows 32 sb + j, chunks 2 cd + h; V^T operand (d block db, 16-key step c):
  // lane p = lane % 16 of group g = lane / 16 (half hh = g / 2, column half dh = g % 2) points at key
  // 16 c + 4 hh + p / 4 (+ 8 for the second read), columns 32 db + 16 dh + 4 (p % 4) .. + 4
  // (the swizzles depend on a row's low 4 / 3 bits only, so the 32-key half sb and the 16-key step c are
  // constant offsets)
  uint32_t kro[8];
#pragma unroll
  for (int cd = 0; cd < 8; ++cd) kro[cd] = (uint32_t)(j * AT_ROW + 16 * k_slot(2 * cd + h, j));
  const int pg = lane & 15, hh = lane >> 5, dh = (lane >> 4) & 1;
  uint32_t vbase[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    const int row = 4 * hh + (pg >> 2);
    const int col = 32 * db + 16 * dh + 4 * (pg & 3);              // bf16 column; 8-byte piece of a chunk
    vbase[db] = (uint32_t)(AT_TILE + row * AT_ROW + 16 * v_slot(col >> 3, row) + 2 * (col & 7));
  }

  v16f_ oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = (v16f_){};
  float m_run = -INFINITY, l_run = 0.0f;

  const int ntiles = (Skv + AT_BN - 1) / AT_BN;
  const int rv_last = Skv - (ntiles - 1) * AT_BN;      // keys in the last tile (1 .. AT_BN)
  issue(0, 0, ntiles == 1 ? rv_last : AT_BN);
  wait_vm_lgkm0<0>();
  barrier_lds();
  // one tile step; LAST (the partial last tile only) masks the keys past Skv. Taking that tile out of the
  // loop keeps the mask out of the full tiles' code: with the uniform test inside the loop the compiler
  // hoisted the 64 per-lane key compares, spilled their masks to VGPR lanes and selected every score in
  // every tile (126 extra VALU instructions per tile).
  auto step = [&](int t, auto last_c) __attribute__((always_inline)) {
    constexpr bool LAST = decltype(last_c)::value;
    const uint8_t* kb = lds + (t & 1) * AT_STAGE;
    if (t + 1 < ntiles) issue(t + 1, (t + 1) & 1, t + 2 == ntiles ? rv_last : AT_BN);
    // S^T for the 32-key halves of the tile (their chains interleaved)
    v16f_ sc[AT_NSB];
#pragma unroll
    for (int sb = 0; sb < AT_NSB; ++sb) sc[sb] = (v16f_){};
#pragma unroll
    for (int cd = 0; cd < 8; ++cd)
#pragma unroll
      for (int sb = 0; sb < AT_NSB; ++sb)
        sc[sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const v8bf*)(kb + sb * 32 * AT_ROW + kro[cd]),
                                                         __builtin_bit_cast(v8bf, qop[cd]), sc[sb], 0, 0, 0);
    if (LAST) {  // keys past Skv: score -inf (lane's key 32 sb + 8 a + 4 h + r)
#pragma unroll
      for (int sb = 0; sb < AT_NSB; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * sb + 8 * (i >> 2) + 4 * h + (i & 3) >= rv_last) sc[sb][i] = -INFINITY;
    }
    // online softmax of tile t (scaled domain: x = s * c_log2); max of the lane's scores as a tree
    float m8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // first level as med3(a, b, 3e38) = max(a, b) for scores below 3e38: fmaxf on raw MFMA results first
      // quiets each input (one v_max x, x per score: 101 max instructions per tile, now 52), med3's results
      // count as quieted, so the levels above need none (a +inf bound is folded back into fmaxf)
      m8[i] = __builtin_amdgcn_fmed3f(sc[0][i], sc[0][i + 8], 3.0e38f);
#pragma unroll
      for (int sb = 1; sb < AT_NSB; ++sb) m8[i] = fmaxf(m8[i], __builtin_amdgcn_fmed3f(sc[sb][i], sc[sb][i + 8], 3.0e38f));
    }
#pragma unroll
    for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
      for (int i = 0; i < w; ++i) m8[i] = fmaxf(m8[i], m8[i + w]);
    const float mx = fmaxf(m8[0], __shfl_xor(m8[0], 32));
    const float x_max = mx * c_log2;
    const bool bump = x_max > m_run;
    const float m_new = bump ? x_max : m_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile (m_run = -inf)
    m_run = m_new;
    float ps[AT_NC];                                     // partial row sums (short dependent chains)
    v4i pop[AT_NC];                                      // p^T operands of the 16-key steps
#pragma unroll
    for (int c = 0; c < AT_NC; ++c) {
      const int sb = c >> 1, r0 = 8 * (c & 1);
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[sb][r0 + e], c_log2, -m_new));
      ps[c] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      pop[c] = (v4i){(int)pack_bf16_pair(p[0], p[1]), (int)pack_bf16_pair(p[2], p[3]),
                     (int)pack_bf16_pair(p[4], p[5]), (int)pack_bf16_pair(p[6], p[7])};
    }
#pragma unroll
    for (int w = AT_NC / 2; w >= 1; w >>= 1)
#pragma unroll
      for (int i = 0; i < w; ++i) ps[i] += ps[i + w];
    const float psum = ps[0];
    l_run = __builtin_fmaf(l_run, alpha, psum);
    if (__builtin_amdgcn_ballot_w64(bump) != 0) {  // wave-uniform: alpha == 1 in lanes that did not move
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
    }
    // O^T += V^T p^T, the V^T operand by two transposing reads (keys 16 c + 4 hh .. + 4 and + 8)
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int c = 0; c < AT_NC; ++c) {
        const v4s_ a0 = lds_read_tr(kb + vbase[db] + 16 * c * AT_ROW);
        const v4s_ a1 = lds_read_tr(kb + vbase[db] + (16 * c + 8) * AT_ROW);
        const v8bf av = __builtin_bit_cast(v8bf, (v4i){__builtin_bit_cast(int, (v2s_){a0[0], a0[1]}),
                                                      __builtin_bit_cast(int, (v2s_){a0[2], a0[3]}),
                                                      __builtin_bit_cast(int, (v2s_){a1[0], a1[1]}),
                                                      __builtin_bit_cast(int, (v2s_){a1[2], a1[3]})});
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(v8bf, pop[c]), oacc[db], 0, 0, 0);
      }
    wait_vm_lgkm0<0>();  // this wave's copies of tile t + 1 have landed
    barrier_lds();       // everyone's have; everyone is done reading tile t's buffer
  };
  const int nfull = rv_last < AT_BN ? ntiles - 1 : ntiles;
  for (int t = 0; t < nfull; ++t) step(t, std::false_type{});
  if (nfull < ntiles) step(nfull, std::true_type{});
  // o = O / l (the two lane halves hold the row sum's two halves)
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (q_ok) {
    uint16_t* op = o + (int64_t)qrow * ldo + head * AT_D;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * db + 8 * a + 4 * h;
        const v16f_& ov = oacc[db];
        *(uint2*)(op + d) = make_uint2(pack_bf16_pair(ov[4 * a] * inv, ov[4 * a + 1] * inv),
                                       pack_bf16_pair(ov[4 * a + 2] * inv, ov[4 * a + 3] * inv));
      }
  }
}

}  // namespace

extern "C" int gwa_dit_attention(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                                 int64_t ldv, void* o, int64_t ldo, int64_t S, int64_t Skv, int64_t heads,
                                 int64_t head_dim, float scale, void* stream) {
  const char* what = "dit_attention";
  GWA_REQUIRE(head_dim == AT_D, "%s: head_dim %lld (only 128 is built)", what, (long long)head_dim);
  GWA_REQUIRE(S >= 0 && Skv > 0 && heads > 0 && heads < 65536, "%s: S=%lld, Skv=%lld, heads=%lld", what,
              (long long)S, (long long)Skv, (long long)heads);
  GWA_REQUIRE(ldq >= heads * AT_D && ldk >= heads * AT_D && ldv >= heads * AT_D && ldo >= heads * AT_D &&
                  ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && ldo % 4 == 0,
              "%s: token strides must be >= heads * 128 (multiples of 8, ldo of 4)", what);
  GWA_REQUIRE(S < (1ll << 31) && Skv < (1ll << 31) && (S + Skv) * (ldq + ldk + ldv + ldo) < (1ll << 46),
              "%s: sizes out of range", what);
  GWA_REQUIRE(scale > 0.0f, "%s: scale must be positive", what);
  GWA_REQUIRE(((Skv - 1) * ldk + heads * AT_D) * 2 < (1ll << 32) && ((Skv - 1) * ldv + heads * AT_D) * 2 < (1ll << 32),
              "%s: k and v must stay below 4 GiB (buffer addressing)", what);
  if (S == 0) return GWA_OK;
  GWA_REQUIRE(q && k && v && o, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(q, 16) && GWA_ALIGNED(k, 16) && GWA_ALIGNED(v, 16) && GWA_ALIGNED(o, 8),
              "%s: q, k, v must be 16-byte aligned, o 8-byte", what);
  const dim3 grid((unsigned)((S + AT_BM - 1) / AT_BM), (unsigned)heads), block(AT_THREADS);
  hipLaunchKernelGGL(dit_attention_kernel, grid, block, 0, (hipStream_t)stream, (const uint16_t*)q, ldq,
                     (const uint16_t*)k, ldk, (const uint16_t*)v, ldv, (uint16_t*)o, ldo, (int)S, (int)Skv,
                     scale * 1.4426950408889634f);
  return gwa_check_launch(what);
}
