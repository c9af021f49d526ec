/*
 * gen_worker_amd — C ABI of the MI355X (gfx950) SVDQuant quantized-linear path.
 *
 * Plain pointers and sizes only; no torch types. Every entry point returns 0
 * on success or a GWA_ERR_* code, and leaves a message for gwa_last_error()
 * (thread-local). Device pointers are HIP device memory; `stream` is a
 * hipStream_t (NULL = the default stream). Nothing synchronizes the host:
 * kernels are enqueued on `stream`, as the reference's Triton launches and
 * torch._scaled_mm run on the current stream.
 *
 * Formats (the int4-g64 / int8 variants of the reference's nvfp4/fp8 path):
 *   bf16/fp16 tensors     : raw 16-bit patterns
 *   int4 packed codes     : uint8 [rows, K/2], two's-complement nibbles,
 *                           element 2j in the LOW nibble (the byte order of
 *                           pack_e2m1, src/gen_worker/models/nvfp4_quant.py:54-56)
 *   int4 group scales     : fp16 [rows, K/64], one per group of 64 along K
 *   int8 codes            : int8 [rows, K]; per-row fp32 scales [rows]
 */
#ifndef GEN_WORKER_AMD_H
#define GEN_WORKER_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  GWA_OK = 0,
  GWA_ERR_INVALID = 1,   /* bad argument / unsupported shape */
  GWA_ERR_HIP = 2,       /* HIP runtime or launch failure */
};

enum { GWA_DT_BF16 = 0, GWA_DT_F16 = 1, GWA_DT_F32 = 2 };

/* GEMM epilogue flags: GELU-tanh after the bias; la given as fp32 (rounded to
 * bf16 in the epilogue, the fp6 GEMMs only) */
enum { GWA_EPI_GELU_TANH = 1, GWA_EPI_LA_F32 = 2 };

/* activation code formats */
enum {
  GWA_QFMT_INT4 = 0, /* uint8 [M, K/2]: two's-complement nibbles, element 2j in the low nibble (the reference
                        contract), written by gwa_svdq_quant_int4 */
  GWA_QFMT_FP6 = 1   /* uint8 [K/128, M, 104] operand records of the fp6 GEMM (see below), written by
                        gwa_svdq_quant_fp6 and gwa_svdq_gemm_w4a4_fp6_next */
};

/* fp6 operand records (activations from gwa_svdq_quant_fp6, weights from
 * gwa_svdq_pack_weight_fp6): stage-major, one 104-byte record per
 * 128-element stage s of K and row r at byte offset (s * rows + r) * 104:
 *   bytes [0, 96)   the stage's two groups as e3m2 codes: element t of group j
 *                   at bits [6t, 6t+6) of bytes [48j, 48j+48) (little-endian)
 *   bytes [96, 100) the two groups' fp16 scales
 *   bytes [100,104) zero (written by every producer: the GEMMs read bytes
 *                   [96, 104) as one (scales, 0) operand pair)
 * (every int4 code -8..7 is an exact e3m2 value). A tile's stage of operand
 * rows is one contiguous run, and its LDS image keeps a bank-conflict-free
 * row stride. The records cover S = ceil(K/128) stages ([K/128, rows, 104]
 * below means [S, rows, 104]): with K % 128 == 64 the last stage is a half
 * stage whose second group holds zero codes (scale 0 from
 * gwa_svdq_pack_weight_fp6, kernel 1's all-zero-group scale from
 * gwa_svdq_quant_fp6), so it adds nothing to a GEMM. */
enum { GWA_FP6_REC = 104 };

/* Readable bytes the fp6 GEMMs need past the last record of each record
 * buffer they read (qa6, qw6): they copy records into LDS in 1 KB runs with
 * scalar offsets the hardware does not range-check, and the run holding a
 * tile's last real row may reach this far past it. Every entry point that
 * takes a record pointer also takes its readable byte count (from the
 * pointer to the end of its storage) and refuses a buffer shorter than the
 * records plus this slack with GWA_ERR_INVALID. */
enum { GWA_FP6_RECORD_SLACK = 1024 };

/* Library version and build description ("archs=gfx950 hip=..."). Mirrors
 * cozy_kernels::build_info, csrc/cozy_kernels/ops.cpp:23-27. */
int gwa_version(void);
const char* gwa_build_info(void);

/* Message for the last failed call on this thread ("" if none). Replaces the
 * TORCH_CHECK / C10_CUDA_KERNEL_LAUNCH_CHECK error surface of
 * csrc/cozy_kernels/probe.cu:15-16,25. */
const char* gwa_last_error(void);

/* Debug build only (libgen_worker_amd_debug.so, compiled with GWA_DEBUG; no
 * reference counterpart: the survey's debug build with bounds checks). Its
 * kernels check the global accesses no hardware range check covers or whose
 * silent drop would hide a mistake — the fp6 GEMMs' 1 KB record copies at
 * scalar offsets (records + GWA_FP6_RECORD_SLACK), kernel 1's record stores,
 * the GEMMs' output stores, the W8A8 copies' K offsets — and a failed check
 * redirects or drops that access and is recorded. This call synchronizes the
 * device, then returns the OR of the sites' bits (bit s = site s of
 * GwaDbgSite in csrc/gwa_common.h: 0/1 activation/weight record copy, 2 fp6
 * output, 3 kernel-1 record, 4 W8A8 copy, 5 W8A8 output) and the first
 * failure (site << 56 | workgroup << 32 | byte offset); clear != 0 resets
 * them. The release library returns GWA_ERR_INVALID. */
int gwa_debug_violations(uint32_t* bits, uint64_t* first, int clear);

/* out[i] = in[i] + 1 for float32 [n]. The extension probe
 * cozy_kernels::probe_add_one, csrc/cozy_kernels/probe.cu:9-27; used by the
 * load-and-probe gate of models/native_kernels.py:120-143. */
int gwa_probe_add_one(const float* in, float* out, int64_t n, void* stream);

/* Kernel 1 — fused activation quantization (+ low-rank down-projection).
 * Replaces cozy_gen_worker::svdq_quant (models/svdq_fused.py:254-306,
 * Triton _quant_smooth_kernel :70-114) plus the separate
 * `la = x2 @ self.proj_down` of models/svdq_fused.py:524.
 *   x          bf16 [M, K] rows with stride ldx (elements), K % 64 == 0
 *   smooth     bf16 [K] or NULL (per-input-channel divisor, 4-bit branch only)
 *   s2         fp32 device scalar or NULL (= 1.0): second-level scale; the
 *              group scale is fp16(amax / (7 * s2)) and codes divide by
 *              (scale * s2), as models/nvfp4_quant.py:98-101 do for nvfp4
 *   proj_down_op  proj_down in MFMA operand order (gwa_svdq_prep_proj_down)
 *              or NULL; rank in {0, 16, 32, 64, 128}
 *   out_format GWA_QFMT_INT4 (q uint8 [M, K/2]); the fp6 records come from
 *              gwa_svdq_quant_fp6
 *   scales     fp16 [M, K/64] (out)
 *   la         bf16 [M, rank] = x @ proj_down on RAW x (out; NULL iff proj_down_op is NULL) */
int gwa_svdq_quant_int4(const void* x, int64_t ldx, const void* smooth, const float* s2,
                        const void* proj_down_op, int64_t rank, int out_format,
                        uint8_t* q, void* scales, void* la,
                        int64_t M, int64_t K, void* stream);

/* proj_down bf16 [K, rank] -> the operand order kernel 1 reads (done once
 * per weight; no reference counterpart: the reference runs x2 @ proj_down
 * as a separate bf16 GEMM, models/svdq_fused.py:524).
 *   out  bf16 [ceil(K/256)*256 * rank] (16-byte aligned), zero padded */
int gwa_svdq_prep_proj_down(const void* proj_down, void* out, int64_t K, int64_t rank, void* stream);

/* Kernel 2 — W4A4 GEMM with the fused SVDQuant epilogue.
 * Replaces _gemm_w4a4 (torch._scaled_mm, models/w4a4.py:173-180) followed by
 * cozy_gen_worker::svdq_epilogue_lora (models/svdq_fused.py:315-377); same
 * math as the registered cozy_gen_worker::svdq_gemm_w4a4_lora
 * (models/svdq_fused.py:180-238, :379-389):
 *   y[m,n] = (sum_g acc_g[m,n] * sa[m,g] * sw[n,g]) * s2 * second[n]
 *            + la[m,:] . up[n,:] + bias[n]          (then optional GELU-tanh)
 *   qa     uint8 [M, K/2]   sa fp16 [M, K/64]
 *   qw     uint8 [N, K/2]   sw fp16 [N, K/64]   (weight [out, in/2] layout)
 *   s2     fp32 device scalar or NULL (= 1.0)
 *   second fp32 [second_numel] (1 or N) or NULL (= 1.0)
 *   la     bf16 [M, rank] or NULL;  up bf16 [N, rank] or NULL; rank in {0, 16, 32, 64, 128}
 *   bias   bf16 [N] or NULL
 *   out    [M, N] of out_dtype (GWA_DT_BF16 or GWA_DT_F16)
 * K % 64 == 0, N % 16 == 0. This is the general path (int8 MFMA on the logical
 * two's-complement weights, any code in [-8, 7]); gwa_svdq_gemm_w4a4_fp6 is
 * the fast path (K % 64 == 0) on fp6 operand records. */
int gwa_svdq_gemm_w4a4(const uint8_t* qa, const void* sa, const uint8_t* qw, const void* sw,
                       const float* s2, const float* second, int64_t second_numel,
                       const void* la, const void* up, int64_t rank, const void* bias,
                       void* out, int out_dtype, int epilogue_flags,
                       int64_t M, int64_t N, int64_t K, void* stream);

/* Debug: exact int32 per-group partial sums out[m, n, g] = sum_{k in g} qx[m,k] qw[n,k]
 * computed by the same MFMA and unpack code as gwa_svdq_gemm_w4a4. No
 * reference counterpart (the reference has no int4 arithmetic); it pins the
 * integer core of kernel 2 bit-exactly. */
int gwa_svdq_group_psums(const uint8_t* qa, const uint8_t* qw, int32_t* out,
                         int64_t M, int64_t N, int64_t K, void* stream);

/* Prepack int4 weights and their group scales as fp6 operand records for
 * gwa_svdq_gemm_w4a4_fp6 (done once per weight; no reference counterpart
 * beyond the layout conversions of models/svdq_layout.py:165-221). Any code
 * in [-8, 7].
 *   qw   uint8 [N, K/2] logical two's-complement codes (in)
 *   sw   fp16 [N, K/64] group scales (in)
 *   qw6  uint8 [K/128, N, 104] records (out); K % 64 == 0. Allocate
 *        GWA_FP6_RECORD_SLACK bytes of slack after it (the GEMMs read up to 1 KB
 *        past and refuse a shorter buffer). */
int gwa_svdq_pack_weight_fp6(const uint8_t* qw, const void* sw, uint8_t* qw6, int64_t N, int64_t K, void* stream);

/* Kernel 2, fp6 path: the contract of gwa_svdq_gemm_w4a4 (replacing
 * _gemm_w4a4 + svdq_epilogue_lora, models/w4a4.py:173-180 and
 * models/svdq_fused.py:315-377) on fp6 operand records: qa6 [K/128, M, 104]
 * from gwa_svdq_quant_fp6, qw6 [K/128, N, 104] from gwa_svdq_pack_weight_fp6
 * (the records carry sa and sw). qa6_bytes / qw6_bytes are the readable
 * bytes from each pointer to the end of its storage: at least the records
 * ((K/128) * M * 104, (K/128) * N * 104) plus GWA_FP6_RECORD_SLACK, else
 * GWA_ERR_INVALID before any launch (operand records are copied in 1 KB runs;
 * the run holding a tile's last real row may reach past them).
 * One exact fp6 MFMA per K-group and 32x32 block. la is bf16 [M, rank], or fp32 with GWA_EPI_LA_F32 in
 * epilogue_flags (rounded to bf16 in the epilogue). K % 64 == 0,
 * N % 16 == 0. */
int gwa_svdq_gemm_w4a4_fp6(const uint8_t* qa6, int64_t qa6_bytes, const uint8_t* qw6, int64_t qw6_bytes,
                           const float* s2, const float* second, int64_t second_numel,
                           const void* la, const void* up, int64_t rank, const void* bias,
                           void* out, int out_dtype, int epilogue_flags,
                           int64_t M, int64_t N, int64_t K, void* stream);

/* Kernel 2 with the next layer's activation quantization fused into the
 * epilogue (config-2 fc1 -> GELU -> fc2). The reference has no kernel for
 * this: it composes Linear -> GELU -> Linear (diffusers FeedForward), i.e.
 * this layer's epilogue (models/svdq_fused.py:315-377) followed by the next
 * layer's svdq_quant (models/svdq_fused.py:293-306) and `la = x2 @
 * proj_down` (:524) on this layer's bf16 output. Here the bf16 output tile
 * never leaves the chip:
 *   y        = this layer's output exactly as gwa_svdq_gemm_w4a4_fp6 computes
 *              it (bf16), also stored to `out` unless out is NULL
 *   next_q6  uint8 [N/128, M, 104] (out): the next layer's fp6 operand
 *            records of y — bit-identical to gwa_svdq_quant_fp6(y,
 *            next_smooth, s2 = NULL, ...). The pointer may
 *            sit inside a larger record buffer of the same M (stage-major:
 *            stage s at byte s * M * 104), e.g. at stage 24 of a [120, M, 104]
 *            buffer whose first stages another producer writes.
 *   next_la_part fp32 [P, M, next_rank] (out), P =
 *            gwa_svdq_gemm_w4a4_fp6_next_partials(M, N): slot p holds
 *            y[:, columns of column tile p] @ proj_down_next[those rows];
 *            gwa_svdq_la_reduce of all of a layer's slots (with other
 *            producers' slots appended, as for [x, y] inputs) gives its bf16
 *            la. NULL iff next_proj_down_op is NULL.
 *   next_smooth       bf16 [N] (the next layer's smoothing factors) or NULL
 *   next_proj_down_op the next layer's proj_down rows for these N inputs in
 *            gwa_svdq_prep_proj_down_fp6 order, next_rank in {0,16,32,64,128}
 * Single-level (the next layer's s2 = 1). Output dtype bf16; la may be fp32
 * (GWA_EPI_LA_F32). qa6_bytes / qw6_bytes as gwa_svdq_gemm_w4a4_fp6 checks
 * them. N % 128 == 0, K % 64 == 0. */
int gwa_svdq_gemm_w4a4_fp6_next(const uint8_t* qa6, int64_t qa6_bytes, const uint8_t* qw6, int64_t qw6_bytes,
                                const float* s2, const float* second, int64_t second_numel,
                                const void* la, const void* up, int64_t rank, const void* bias,
                                void* out, int epilogue_flags,
                                const void* next_smooth, const void* next_proj_down_op, int64_t next_rank,
                                uint8_t* next_q6, float* next_la_part,
                                int64_t M, int64_t N, int64_t K, void* stream);

/* Number of la partial slots gwa_svdq_gemm_w4a4_fp6_next writes (its column
 * tiles) for M rows and N outputs. */
int64_t gwa_svdq_gemm_w4a4_fp6_next_partials(int64_t M, int64_t N);

/* The output tile gwa_svdq_gemm_w4a4_fp6 uses for M rows and N outputs
 * (GWA_FP6_TILE_*; -1 for an empty shape). No reference counterpart: the
 * reference's Triton GEMM autotunes its tile (models/svdq_fused.py:157-178). */
enum {
  GWA_FP6_TILE_256x256 = 0, GWA_FP6_TILE_256x128 = 1, GWA_FP6_TILE_128x128 = 2, GWA_FP6_TILE_192x256 = 3,
  GWA_FP6_TILE_288x192 = 4, GWA_FP6_TILE_256x192 = 5, GWA_FP6_TILE_64x128 = 6
};
int gwa_svdq_gemm_w4a4_fp6_tile(int64_t M, int64_t N);

/* Test and tuning hook: every later gwa_svdq_gemm_w4a4_fp6 (and the one-call
 * linears) uses this tile instead of the model's choice (-1 restores the
 * model; the next-layer GEMM keeps its own 256-row tiles). Process-wide;
 * returns the previous setting. */
int gwa_svdq_gemm_w4a4_fp6_force_tile(int tile);

/* Kernel 1 for the fp6 GEMM lane: the arithmetic of gwa_svdq_quant_int4
 * (same codes and scales, bit for bit) written as fp6 operand records, with
 * the low-rank product as fp32 partial sums (replaces
 * cozy_gen_worker::svdq_quant, models/svdq_fused.py:293-306, plus
 * `la = x2 @ proj_down`, :524):
 *   x          bf16 [M, K] rows with stride ldx (elements), K % 64 == 0 (a
 *              half stage reads no column past K)
 *   smooth     bf16 [K] or NULL;  s2 fp32 device scalar or NULL (= 1.0)
 *   proj_down_op6  proj_down in this kernel's operand order
 *              (gwa_svdq_prep_proj_down_fp6) or NULL; rank in {0,16,32,64,128}
 *   q6         uint8 [K/128, M, 104] records (out). The pointer may sit inside
 *              a larger record buffer of the same M (stage s at byte s*M*104):
 *              a layer whose input concatenates [x, other] takes its first
 *              K/128 stages from here and the rest from another producer
 *              (gwa_svdq_gemm_w4a4_fp6_next).
 *   la_part    fp32 [P, M, rank] (out), P = gwa_svdq_quant_fp6_partials(M, K,
 *              rank): partial sums of x @ proj_down on RAW x over P ranges of
 *              K, every slot fully written; gwa_svdq_la_reduce sums them into
 *              the bf16 la (a fixed order: deterministic). NULL iff
 *              proj_down_op6 is NULL. */
int gwa_svdq_quant_fp6(const void* x, int64_t ldx, const void* smooth, const float* s2,
                       const void* proj_down_op6, int64_t rank, uint8_t* q6, float* la_part,
                       int64_t M, int64_t K, void* stream);

/* Number of la partial slots gwa_svdq_quant_fp6 writes for this shape (0 for
 * rank 0 or a bad shape). */
int64_t gwa_svdq_quant_fp6_partials(int64_t M, int64_t K, int64_t rank);

/* Kernel 1 for the fp6 lane with la written as bf16 (replaces
 * cozy_gen_worker::svdq_quant, models/svdq_fused.py:293-306, plus
 * `la = x2 @ proj_down`, :524, in one call): gwa_svdq_quant_fp6 into the
 * partial slots in la_ws, then gwa_svdq_la_reduce into la bf16 [M, rank]
 * (rank in {16,32,64,128}). la_ws_bytes must be at least
 * gwa_svdq_quant_fp6_la_workspace(M, K, rank). */
int gwa_svdq_quant_fp6_la(const void* x, int64_t ldx, const void* smooth, const float* s2,
                          const void* proj_down_op6, int64_t rank, uint8_t* q6, void* la, float* la_ws,
                          int64_t la_ws_bytes, int64_t M, int64_t K, void* stream);

/* Bytes of la workspace gwa_svdq_quant_fp6_la needs for this shape (0 for a
 * bad shape). */
int64_t gwa_svdq_quant_fp6_la_workspace(int64_t M, int64_t K, int64_t rank);

/* la bf16 [M, rank] = RN_bf16(part[0] + part[1] + ... + part[P-1]) (fp32
 * additions in that order; part fp32 [P, M, rank], rank % 16 == 0): the
 * bf16 la of the reference's `x2 @ proj_down` (models/svdq_fused.py:524)
 * from the producers' partial sums. */
int gwa_svdq_la_reduce(const float* part, int64_t P, int64_t M, int64_t rank, void* la, void* stream);

/* proj_down bf16 [K, rank] -> the operand order of gwa_svdq_quant_fp6 and of
 * the next-layer epilogue of gwa_svdq_gemm_w4a4_fp6_next (done once per
 * weight; no reference counterpart). K % 64 == 0.
 *   out  bf16 [ceil(K/128) * 128 * rank] (16-byte aligned; a half stage's rows
 *        past K are zeros): stage-major, element
 *        (((s*4 + j)*(rank/16) + b)*64 + l)*8 + e = proj_down[128s + 32(l/16) + 8j + e][16b + l%16] */
int gwa_svdq_prep_proj_down_fp6(const void* proj_down, void* out, int64_t K, int64_t rank, void* stream);

/* Debug: exact int32 per-group partial sums (layout of gwa_svdq_group_psums)
 * through the fp6 GEMM's MFMA on fp6 operand records. No reference
 * counterpart. This kernel reads records through range-checked lane offsets:
 * qa6_bytes / qw6_bytes must cover the records, no slack. */
int gwa_svdq_group_psums_fp6(const uint8_t* qa6, int64_t qa6_bytes, const uint8_t* qw6, int64_t qw6_bytes,
                             int32_t* out, int64_t M, int64_t N, int64_t K, void* stream);

/* One whole SVDQuant W4A4 linear on the fp6 lane: the forward of the
 * reference's fused module, _SvdqFusedLinear.forward
 * (models/svdq_fused.py:516-527: svdq_quant -> _gemm_w4a4 -> x2 @ proj_down
 * -> svdq_epilogue_lora), as one call: gwa_svdq_quant_fp6 (records + la
 * partial slots), gwa_svdq_la_reduce and gwa_svdq_gemm_w4a4_fp6, enqueued on
 * `stream`. Arguments as those entry points take them:
 *   x        bf16 [M, K] rows with stride ldx; smooth bf16 [K] or NULL;
 *            s2 fp32 device scalar or NULL (= 1.0)
 *   proj_down_op6  gwa_svdq_prep_proj_down_fp6 order, or NULL (rank 0);
 *            proj_up bf16 [N, rank] (NULL iff proj_down_op6 is NULL)
 *   qw6      the weight's fp6 records (gwa_svdq_pack_weight_fp6) and
 *            qw6_bytes, its readable bytes: >= (K/128) * N * 104 +
 *            GWA_FP6_RECORD_SLACK (the activation records live in the
 *            workspace, slack included)
 *   second / bias / out / out_dtype as gwa_svdq_gemm_w4a4_fp6; epilogue_flags
 *            GWA_EPI_GELU_TANH or 0
 *   workspace  device memory of workspace_bytes >=
 *            gwa_svdq_w4a4_linear_fp6_workspace(M, K, rank), 256-byte aligned:
 *            the activation records (+ slack), the la partial slots and the
 *            bf16 la. Nothing in it needs to be initialised; it must not be
 *            reused by another call until this call's work on `stream` ends.
 * K % 64 == 0, N % 16 == 0. */
int gwa_svdq_w4a4_linear_fp6(const void* x, int64_t ldx, const void* smooth, const float* s2,
                             const void* proj_down_op6, int64_t rank, const uint8_t* qw6, int64_t qw6_bytes,
                             const float* second, int64_t second_numel, const void* proj_up,
                             const void* bias, void* out, int out_dtype, int epilogue_flags,
                             int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                             void* stream);

/* Workspace bytes gwa_svdq_w4a4_linear_fp6 needs for M rows, K inputs and
 * this rank (0 for an unsupported shape). */
int64_t gwa_svdq_w4a4_linear_fp6_workspace(int64_t M, int64_t K, int64_t rank);

/* Size of the static scratch of gwa_svdq_w4a4_linear_fp6_noalloc (128 MiB). */
enum { GWA_NOALLOC_SCRATCH_MIB = 128 };
#define GWA_NOALLOC_SCRATCH_BYTES ((int64_t)GWA_NOALLOC_SCRATCH_MIB << 20)

/* gwa_svdq_w4a4_linear_fp6 without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * Its intermediates live in a static device array of
 * GWA_NOALLOC_SCRATCH_BYTES inside this library (one copy per GPU, held
 * until the process ends); a shape whose
 * gwa_svdq_w4a4_linear_fp6_workspace(M, K, rank) exceeds it is refused with
 * GWA_ERR_INVALID before anything is enqueued (at rank 32: K = 3072 fits up
 * to 40,329 rows, K = 12288 up to 10,229, K = 15360 up to 8,191, so every
 * linear of the 4608-token Flux-shaped DiT fits). Calls no hipMalloc, hipFree or
 * other allocating routine. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams or threads without
 * ordering between them) race. Nothing in the array needs to start at zero
 * (every byte a call reads back was written earlier in the same call). Call it
 * with the stream's device current. Same arguments and results as
 * gwa_svdq_w4a4_linear_fp6. */
int gwa_svdq_w4a4_linear_fp6_noalloc(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                     const void* proj_down_op6, int64_t rank, const uint8_t* qw6, int64_t qw6_bytes,
                                     const float* second, int64_t second_numel, const void* proj_up,
                                     const void* bias, void* out, int out_dtype, int epilogue_flags,
                                     int64_t M, int64_t N, int64_t K, void* stream);

/* GWA_NOALLOC_SCRATCH_BYTES, as the built library sees it. */
int64_t gwa_svdq_w4a4_linear_fp6_noalloc_scratch_bytes(void);

/* One whole SVDQuant W4A4 linear for a few tokens: the forward of
 * _SvdqFusedLinear (models/svdq_fused.py:516-527) at the token counts of the
 * DiT's adaLN modulation linears (one token per image), where the GEMM tiles
 * would spend 32-128 rows of work on each real one. Streams the int4 weight
 * in the reference's layout (the module's `weight` uint8 [N, K/2], two's-
 * complement nibbles, low nibble = even input; `weight_scale` fp16 [N, K/64])
 * once; kernel 1 (gwa_svdq_quant_fp6) supplies la's partial slots when rank >
 * 0, and the GEMV quantizes the rows itself with kernel 1's quantizer (codes
 * and scales bit-identical). Same group order and epilogue as the GEMM
 * (acc = fma(P_g, sx_g * sw_g, acc), * s2 * second, + la . up, + bias,
 * optional GELU-tanh); only the low-rank sum rounds differently.
 *   x / smooth / s2 / proj_down_op6 / proj_up / second / bias / out /
 *   out_dtype / epilogue_flags as gwa_svdq_w4a4_linear_fp6
 *   qw uint8 [N, K/2] (16-byte aligned rows), sw fp16 [N, K/64]
 *   workspace >= gwa_svdq_w4a4_linear_gemv_workspace(M, K, rank) bytes,
 *   256-byte aligned, nothing in it needs initialising
 * 1 <= M <= gwa_svdq_w4a4_gemv_max_m(K, rank), K % 128 == 0, N % 16 == 0. */
int gwa_svdq_w4a4_linear_gemv(const void* x, int64_t ldx, const void* smooth, const float* s2,
                              const void* proj_down_op6, int64_t rank, const uint8_t* qw, const void* sw,
                              const float* second, int64_t second_numel, const void* proj_up, const void* bias,
                              void* out, int out_dtype, int epilogue_flags, int64_t M, int64_t N, int64_t K,
                              void* workspace, int64_t workspace_bytes, void* stream);

/* The most tokens gwa_svdq_w4a4_linear_gemv takes at this K and rank (up to
 * 8; 0 if K % 128 != 0, K > 8192 or the rank is unsupported). */
int gwa_svdq_w4a4_gemv_max_m(int64_t K, int64_t rank);

/* Workspace bytes of gwa_svdq_w4a4_linear_gemv (0 for an unsupported shape). */
int64_t gwa_svdq_w4a4_linear_gemv_workspace(int64_t M, int64_t K, int64_t rank);

/* Standalone epilogue: out = y0 * (s2 * second) + la @ up^T + bias (bf16 out).
 * cozy_gen_worker::svdq_epilogue_lora, models/svdq_fused.py:315-377.
 *   y0 bf16 [M, N]; la bf16 [M, rank]; up bf16 [N, rank]; bias bf16 [N] or NULL */
int gwa_svdq_epilogue_lora(const void* y0, const void* la, const void* up, int64_t rank,
                           const float* s2, const float* second, int64_t second_numel,
                           const void* bias, void* out, int64_t M, int64_t N, void* stream);

/* W8A8 per-token int8 activation quantization.
 * Replaces the quantizer of _Fp8ScaledLinear.forward (models/w8a8.py:259-297,
 * :363) with the reference's int8 formula (models/svdq_layout.py:261-275,
 * block = one row): sa = max(amax/127, 1e-12); q = clamp(rne(x/sa), -127, 127).
 *   x bf16 [M, K] (row stride ldx) -> q int8 [M, K], sa fp32 [M] */
int gwa_w8a8_quant_int8(const void* x, int64_t ldx, int8_t* q, float* sa,
                        int64_t M, int64_t K, void* stream);

/* W8A8 activation quantization in the reference's three modes: quantize(x2,
 * pertensor, static) of models/w8a8.py:261-273 with the int8 formula above.
 *   input_scale != NULL (static, the layer's input_scale buffer [1, 1] fp32):
 *       sa = input_scale[0] unchanged; sa is [1] if pertensor, else [M] (the
 *       reference's static.expand(M, 1));
 *   input_scale == NULL, pertensor: sa [1] = max(amax(|x|)/127, 1e-12) over
 *       the whole tensor; amax_ws is 4 bytes of device memory the call uses;
 *   input_scale == NULL, !pertensor: per token, as gwa_w8a8_quant_int8.
 *   q = clamp(rne(x / sa), -127, 127). */
int gwa_w8a8_quant(const void* x, int64_t ldx, int8_t* q, float* sa, const float* input_scale, int pertensor,
                   uint32_t* amax_ws, int64_t M, int64_t K, void* stream);

/* Kernel 3 — W8A8 GEMM with per-token (sa_numel == M) or per-tensor
 * (sa_numel == 1) activation scales and per-channel weight scales.
 * Replaces torch._scaled_mm(xq, W.t(), scale_a=sa, scale_b=weight_scale.t(),
 * bias, out_dtype) of models/w8a8.py:374-378, and the pertensor branch
 * (:366-372) with its weight scale and bias fused in fp32:
 *   y[m,n] = (sum_k qa[m,k] qw[n,k]) * sa[m or 0] * sw[n] + bias[n]
 *   qa int8 [M, K]; qw int8 [N, K]; sa fp32 [M] or [1]; sw fp32 [N]
 *   bias of bias_dtype [N] or NULL; out [M, N] of out_dtype (bf16/f16)
 * K % 64 == 0, N % 16 == 0, N < 2^21. */
int gwa_w8a8_gemm(const int8_t* qa, const int8_t* qw, const float* sa, int64_t sa_numel, const float* sw,
                  const void* bias, int bias_dtype, void* out, int out_dtype,
                  int64_t M, int64_t N, int64_t K, void* stream);

/* The output tile gwa_w8a8_gemm uses for this shape (GWA_W8A8_TILE_*; -1 for
 * an empty shape): 256 x 256 tiles (direct-to-LDS copies, 512 threads; K a
 * multiple of 128) when their rounds over the CUs finish before those of
 * 128 x 128 tiles, else 128 x 128. No reference counterpart: torch._scaled_mm
 * picks its own kernel. */
enum { GWA_W8A8_TILE_128x128 = 0, GWA_W8A8_TILE_256x256 = 1 };
int gwa_w8a8_gemm_tile(int64_t M, int64_t N, int64_t K);

/* Test and tuning hook: every later gwa_w8a8_gemm uses this tile (-1
 * restores the choice above; K % 128 != 0 or K >= 2^23 always takes
 * 128 x 128). Process-wide; returns the previous setting. */
int gwa_w8a8_gemm_force_tile(int tile);

/* AWQ W4A16 linear (the M = 1 adaLN modulation layers).
 * Replaces cozy_gen_worker::awq_w4a16_mm (models/svdq_awq_packed.py:48-115;
 * schema "(Tensor x2, Tensor weight, Tensor wscales, Tensor wzeros, Tensor? bias) -> Tensor"):
 *   y[m, n] = sum_k RN_bf16(code[n, k] * wscales[n, k/64] + wzeros[n, k/64]) * x[m, k] + bias[n]
 * in fp32, rounded to bf16.
 *   x bf16 [M, K] (row stride ldx, 16-byte aligned); weight uint8 [N, K/2] (code of column 2j in the
 *   low nibble of byte j, 0..15); wscales, wzeros bf16 [N, K/64]; bias bf16 [N] or NULL; out bf16 [M, N].
 * N % 16 == 0, K % 128 == 0 (models/svdq_awq_packed.py:23-24), K <= 32768. */
int gwa_awq_w4a16_mm(const void* x, int64_t ldx, const void* weight, const void* wscales, const void* wzeros,
                     const void* bias, void* out, int64_t M, int64_t N, int64_t K, void* stream);

/* AWQ W4A16 weight -> bf16 [N, K] (16-byte aligned), the values gwa_awq_w4a16_mm multiplies by:
 * the dequantized weight of the reference's decode path (models/svdq_awq.py:74-82, rounded to bf16 as
 * decode_awq_linear's copy into a bf16 Linear does, :112-114). For callers with many activation rows
 * (a library GEMM follows). K % 64 == 0. */
int gwa_awq_w4a16_dequant(const void* weight, const void* wscales, const void* wzeros, void* out,
                          int64_t N, int64_t K, void* stream);

/* nvfp4 compatibility lane (the reference's modelopt nvfp4 contract: e2m1
 * codes, element 2j in the low nibble; e4m3 scales per block of 16 along K;
 * a second-level fp32 scale). Scale grids [rows, K/16] are flat or in the
 * cuBLAS 128 x 4 blocked order of to_blocked_scales
 * (models/nvfp4_quant.py:72-84), whose size is
 * gwa_nvfp4_blocked_scale_numel(rows, K/16) (blocked_scale_numel, :87-89). */
enum { GWA_NVFP4_SCALES_FLAT = 0, GWA_NVFP4_SCALES_BLOCKED = 1 };

int64_t gwa_nvfp4_blocked_scale_numel(int64_t rows, int64_t kblocks);

/* Activation quantization, bit-identical to quantize_activation_torch
 * (models/nvfp4_quant.py:92-103; the op cozy_gen_worker::quant_nvfp4_act,
 * :185-187):
 *   x       bf16 [M, K] rows with stride ldx (elements), K % 16 == 0
 *   s2      fp32 device scalar: the second-level scale
 *   q       uint8 [M, K/2] codes (out)
 *   scales  e4m3 bytes (out): flat [M, K/16] or blocked (only the real
 *           entries are written; the caller zeroes the padding)
 *   xdq     bf16 [M, K] (out, or NULL): code * e4m3 scale (exact), the
 *           operand of the lane's bf16 GEMM (torch._scaled_mm's product,
 *           models/w4a4.py:173-180, without s2) */
int gwa_nvfp4_quant_act(const void* x, int64_t ldx, const float* s2, uint8_t* q, uint8_t* scales,
                        int scale_layout, void* xdq, int64_t M, int64_t K, void* stream);

/* gwa_nvfp4_quant_act with the forward's dynamic second-level scale
 * (models/w4a4.py:342-343: s2 = max(max|x| / (6 * 448), 1e-12), fp32)
 * computed on the device: a first pass writes per-workgroup maxima into
 * parts (fp32 scratch of 1024 values), the quantizer folds them and also
 * writes s2 to s2_out (fp32 device scalar) for the epilogue. NaN inputs are
 * not supported. */
int gwa_nvfp4_quant_act_dyn(const void* x, int64_t ldx, float* s2_out, float* parts, uint8_t* q,
                            uint8_t* scales, int scale_layout, void* xdq, int64_t M, int64_t K, void* stream);

/* codes uint8 [rows, K/2] + e4m3 scales (flat or blocked) -> bf16 [rows, K]
 * = code * scale, exact (dequantize_nvfp4_tensor, models/w4a4.py:157-164,
 * without the second-level scale). */
int gwa_nvfp4_dequant(const uint8_t* q, const uint8_t* scales, int scale_layout, void* out, int64_t rows,
                      int64_t K, void* stream);

/* The module's epilogue after the bf16 GEMM (_W4A4Linear.forward,
 * models/w4a4.py:349-351), in place on y bf16 [M, N] (N % 8 == 0):
 * y = RN_bf16(RN_bf16(y * c) + bias), c = RN_bf16(s2 * ws2) (s2, ws2 fp32
 * device scalars; bias bf16 [N] or NULL), each step rounded as torch's bf16
 * multiply and add round. */
int gwa_nvfp4_scale_bias(void* y, const float* s2, const float* ws2, const void* bias, int64_t M, int64_t N,
                         void* stream);

/* Row-major 2-D transpose of 1/2/4-byte elements: dst[c, r] = src[r, c].
 * Layout plumbing for the reference's K-major operands (wq_kn [K/2, N] of
 * models/svdq_fused.py:214, proj_down [in, rank] of :506-507). */
int gwa_transpose_2d(const void* src, void* dst, int64_t rows, int64_t cols,
                     int64_t elem_size, void* stream);

/* ---- Block glue of the benchmark's Flux-shaped DiT (config 4) ----------------
 * No counterpart among the reference's entry points: the reference's DiT is
 * diffusers' FluxTransformerBlock / FluxSingleTransformerBlock, which computes
 * these with torch ops between its (quantized) linears. Each is one pass with
 * the torch expression's bf16 roundings; all tensors bf16, rows with strides. */

/* q and k of one token range -> RMSNorm over head_dim (sum of squares in fp32,
 * rsqrt(mean + eps), rounded to bf16, times the bf16 weight wq / wk [128])
 * -> rotary embedding on interleaved (even, odd) pairs with the bf16 tables
 * cos_t / sin_t [table_rows, 64] at positions pos0 + row; v (xv, optional)
 * copied to ov. Inputs [rows, heads * 128] at row stride ldx (e.g. column
 * slices of a fused qkv output), outputs at row stride ldo. head_dim == 128. */
int gwa_dit_qk_norm_rope(const void* xq, const void* xk, const void* xv, int64_t ldx, const void* wq,
                         const void* wk, const void* cos_t, const void* sin_t, int64_t pos0, int64_t table_rows,
                         void* oq, void* ok, void* ov, int64_t ldo, int64_t rows, int64_t heads, int64_t head_dim,
                         float eps, void* stream);

/* out = RN(RN(RN(LayerNorm(x)) * RN(1 + scale)) + shift): LayerNorm without
 * affine over cols (fp32 mean and biased variance), scale / shift bf16
 * [cols]; cols a multiple of 512, <= 4096; 16-byte aligned rows. */
int gwa_dit_adaln_modulate(const void* x, int64_t ldx, const void* scale, const void* shift, void* out,
                           int64_t ldo, int64_t rows, int64_t cols, float eps, void* stream);

/* out = RN(x + RN(gate * y)), gate bf16 [cols] broadcast over rows; out may
 * be x. cols % 8 == 0, 16-byte aligned rows. */
int gwa_dit_gate_residual(const void* x, int64_t ldx, const void* y, int64_t ldy, const void* gate, void* out,
                          int64_t ldo, int64_t rows, int64_t cols, void* stream);

/* Softmax attention without a mask (the DiT's joint self-attention; the
 * scaled_dot_product_attention diffusers' FluxAttnProcessor calls): for every
 * head h and query s, o[s][h] = sum_t softmax_t(q[s][h] . k[t][h] * scale)
 * v[t][h], fp32 accumulation, bf16 q / k / v / o as rows [token][head][128]
 * with token strides ldq / ldk / ldv / ldo (elements). One pass over the keys
 * with an online softmax; p is rounded to bf16 for the p v product.
 * head_dim == 128, Skv >= 1, q / k / v 16-byte aligned. */
int gwa_dit_attention(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, void* o,
                      int64_t ldo, int64_t S, int64_t Skv, int64_t heads, int64_t head_dim, float scale,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GEN_WORKER_AMD_H */
