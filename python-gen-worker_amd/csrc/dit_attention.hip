// Attention of the benchmark's Flux-shaped DiT (joint [text; image] self-attention, no mask, head_dim 128,
// bf16 in and out): softmax(q k^T / sqrt(128)) v per head in one pass over the keys with an online softmax
// (the flash-attention recurrence), in place of torch's scaled_dot_product_attention (which diffusers'
// FluxAttnProcessor calls; here the vendor kernel ran at ~0.49 PFLOP/s).
//
// Work split: a 256-thread workgroup owns 128 queries of one head (4 waves x 32 queries) and walks the keys
// in tiles of 64. Per tile, K [64 keys][128] and V transposed [128][64 keys] are staged in LDS (double
// buffered; the next tile's global loads are issued before the current tile's MFMAs and written to the other
// buffers after them, one barrier per tile). Each wave computes, with bf16 MFMA 32x32x16 and fp32
// accumulation:
//   S^T = K_tile q^T            (keys x queries: a lane holds one query and 16 keys of each 32-key half)
//   p   = exp2(S * c - m)       (c = log2(e) / sqrt(128), m the query's running max: the two lane halves
//                                exchange their maxima; O is rescaled only in tiles where some lane's max
//                                moved; the row sums stay per lane until the end)
//   O^T = O^T * exp2(m_old - m) + V^T p^T   (head_dim x queries: a lane holds one query's 64 outputs)
// The key order inside a 16-key MFMA step is the one S^T's output layout leaves p in, and V^T is read in the
// same order, so p goes from the S MFMA to the O MFMA without leaving registers. Output o = O / l in bf16,
// written as rows [query][head][128] (the layout the next linear reads).
#include "gwa_common.h"

namespace {

constexpr int AT_D = 128, AT_BM = 128, AT_BN = 64, AT_THREADS = 256;
constexpr int AT_KROW = AT_D * 2 + 16;                 // K tile row bytes (272: conflict-free 16-byte reads)
constexpr int AT_VROW = AT_BN * 2 + 16;                // V^T tile row bytes (144: conflict-free 16-byte reads)
constexpr int AT_KBYTES = AT_BN * AT_KROW;             // 17408
constexpr int AT_VBYTES = AT_D * AT_VROW;              // 18432
constexpr int AT_STAGE = AT_KBYTES + AT_VBYTES;
constexpr int AT_LDS = 2 * AT_STAGE;                   // 71680

typedef float v16f_ __attribute__((ext_vector_type(16)));
constexpr float kLazy = 0.0f;   // log2 headroom of the running max before it moves (0: the exact running max)

__device__ __forceinline__ uint32_t pack_bf16_pair(float a, float b) { return pack_bf16x2_rn(a, b); }

__global__ __launch_bounds__(AT_THREADS, 2) void dit_attention_kernel(
    const uint16_t* __restrict__ q, int64_t ldq, const uint16_t* __restrict__ k, int64_t ldk,
    const uint16_t* __restrict__ v, int64_t ldv, uint16_t* __restrict__ o, int64_t ldo, int S, int Skv,
    float c_log2) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[AT_LDS];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
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

  // staging of one key tile: K rows (tid: 4 chunks of 16 bytes of [64 keys][128]), V^T (a lane takes two
  // keys 2p, 2p+1 and two 8-column chunks, writes key-pair dwords into V^T rows). Buffer loads: each lane's
  // offsets are fixed, the tile's rows come in through the scalar offset.
  const rsrc_t kbuf = make_rsrc(k, (uint32_t)(((int64_t)(Skv - 1) * ldk + gridDim.y * AT_D) * 2));
  const rsrc_t vbuf = make_rsrc(v, (uint32_t)(((int64_t)(Skv - 1) * ldv + gridDim.y * AT_D) * 2));
  v4i kreg[4], vreg[4];
  const int vp = lane & 31;                            // key pair of this lane
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = u * AT_THREADS + tid;                // K chunk: key c / 16, columns 8 (c % 16) ..
    koff[u] = (uint32_t)(((c >> 4) * ldk + head * AT_D + 8 * (c & 15)) * 2);
    // V: key 2vp + (u & 1), 8-column chunk 4 wave + h + 2 (u >> 1)
    voff[u] = (uint32_t)(((2 * vp + (u & 1)) * ldv + head * AT_D + 8 * (4 * wave + h + 2 * (u >> 1))) * 2);
  }
  auto load_k = [&](int t) __attribute__((always_inline)) {
    const uint32_t ks = (uint32_t)((int64_t)t * AT_BN * ldk * 2);
#pragma unroll
    for (int u = 0; u < 4; ++u) kreg[u] = __builtin_amdgcn_raw_buffer_load_b128(kbuf, koff[u], ks, 0);
  };
  auto load_v = [&](int t) __attribute__((always_inline)) {
    const uint32_t vs = (uint32_t)((int64_t)t * AT_BN * ldv * 2);
#pragma unroll
    for (int u = 0; u < 4; ++u) vreg[u] = __builtin_amdgcn_raw_buffer_load_b128(vbuf, voff[u], vs, 0);
  };
  // V^T key positions: bits 2 and 3 of a key's index in the tile swapped, so the 8 keys of a lane's 16-key
  // MFMA step (16c + 4h + 0..3 and 16c + 8 + 4h + 0..3) sit at 16c + 8h + 0..7: one 16-byte read
  const uint32_t vpos = (uint32_t)(((2 * vp) & ~12) | (((2 * vp) & 4) << 1) | (((2 * vp) & 8) >> 1)) * 2;
  // LDS: K buffers 0, 1, then V^T buffers 0, 1
  auto kbuf_at = [&](int b) __attribute__((always_inline)) { return lds + b * AT_KBYTES; };
  auto vbuf_at = [&](int b) __attribute__((always_inline)) { return lds + 2 * AT_KBYTES + b * AT_VBYTES; };
  auto store_k = [&](int b) __attribute__((always_inline)) {
    uint8_t* kb = kbuf_at(b);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = u * AT_THREADS + tid;
      *(v4i*)(kb + (c >> 4) * AT_KROW + 16 * (c & 15)) = kreg[u];
    }
  };
  auto store_v = [&](int b) __attribute__((always_inline)) {
    uint8_t* vb = vbuf_at(b);
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const v4i a = vreg[2 * cc], bb = vreg[2 * cc + 1];  // keys 2vp, 2vp + 1 of columns 8 (4 wave + h + 2 cc) ..
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = __builtin_amdgcn_perm((uint32_t)bb[e], (uint32_t)a[e], 0x05040100u);  // column 2e
        const uint32_t hi = __builtin_amdgcn_perm((uint32_t)bb[e], (uint32_t)a[e], 0x07060302u);  // column 2e+1
        const int col = 8 * (4 * wave + h + 2 * cc) + 2 * e;
        *(uint32_t*)(vb + col * AT_VROW + vpos) = lo;
        *(uint32_t*)(vb + (col + 1) * AT_VROW + vpos) = hi;
      }
    }
  };
  // S^T of one key tile (the two 32-key halves' MFMA chains interleaved)
  auto s_tile = [&](int b, v16f_* s) __attribute__((always_inline)) {
    s[0] = (v16f_){};
    s[1] = (v16f_){};
    const uint8_t* kr = kbuf_at(b) + j * AT_KROW + 16 * h;
#pragma unroll
    for (int cd = 0; cd < 8; ++cd)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
        s[sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const v8bf*)(kr + 32 * sb * AT_KROW + 32 * cd),
                                                        __builtin_bit_cast(v8bf, qop[cd]), s[sb], 0, 0, 0);
  };

  v16f_ oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = (v16f_){};
  float m_run = -INFINITY, l_run = 0.0f;

  // Iteration t: tile t+1's global loads go out first, tile t's S, softmax and p v run on the LDS copies,
  // then tile t+1 is written into the other buffers (last read in iteration t-1) and one barrier follows.
  const int ntiles = Skv / AT_BN;
  load_k(0);
  load_v(0);
  store_k(0);
  store_v(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    if (t + 1 < ntiles) {
      load_k(t + 1);
      load_v(t + 1);
    }
    v16f_ sc[2];
    s_tile(t & 1, sc);
    // online softmax of tile t (scaled domain: x = s * c_log2); max of the lane's 32 scores as a tree
    float m8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) m8[i] = fmaxf(fmaxf(sc[0][i], sc[0][i + 8]), fmaxf(sc[1][i], sc[1][i + 8]));
#pragma unroll
    for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
      for (int i = 0; i < w; ++i) m8[i] = fmaxf(m8[i], m8[i + w]);
    const float mx = fmaxf(m8[0], __shfl_xor(m8[0], 32));
    // the running max moves when a score exceeds it by more than kLazy (log2 units; p <= 2^kLazy otherwise,
    // and O and l share the reference, so o = O / l does not depend on it); O is rescaled only then
    const float x_max = mx * c_log2;
    const bool bump = x_max > m_run + kLazy;
    const float m_new = bump ? x_max : m_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile (m_run = -inf)
    m_run = m_new;
    float ps[4];                                         // four partial row sums (short dependent chains)
    v4i pop[4];                                          // p^T operands of the four 16-key steps
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int sb = c >> 1, r0 = 8 * (c & 1);
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[sb][r0 + e], c_log2, -m_new));
      ps[c] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      pop[c] = (v4i){(int)pack_bf16_pair(p[0], p[1]), (int)pack_bf16_pair(p[2], p[3]),
                     (int)pack_bf16_pair(p[4], p[5]), (int)pack_bf16_pair(p[6], p[7])};
    }
    const float psum = (ps[0] + ps[1]) + (ps[2] + ps[3]);
    l_run = __builtin_fmaf(l_run, alpha, psum);
    if (__builtin_amdgcn_ballot_w64(bump) != 0) {  // wave-uniform: alpha == 1 in lanes that did not move
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
    }
    // O^T += V^T p^T: V^T row d = 32 db + j, positions 16 c + 8 h .. + 8 (keys 16 c + 4 h .. + 4 and
    // 16 c + 8 + 4 h .. + 4)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const uint8_t* vr = vbuf_at(t & 1) + (32 * db + j) * AT_VROW + 16 * h;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const v8bf*)(vr + 32 * c),
                                                           __builtin_bit_cast(v8bf, pop[c]), oacc[db], 0, 0, 0);
    }
    if (t + 1 < ntiles) {
      store_k((t + 1) & 1);
      store_v((t + 1) & 1);
    }
    __syncthreads();
  }
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
  GWA_REQUIRE(S >= 0 && Skv > 0 && Skv % AT_BN == 0 && heads > 0 && heads < 65536,
              "%s: S=%lld, Skv=%lld (a positive multiple of %d), heads=%lld", what, (long long)S, (long long)Skv,
              AT_BN, (long long)heads);
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
