"""CPU oracle for the SVDQuant int4-g64 / W8A8 int8 quantized-linear path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker. The product (``gen_worker_amd``) never imports it and has no CPU
fallback.

What this restates
------------------
The reference (cozy-creator/python-gen-worker) implements the quantized-linear
path in nvfp4 (e2m1 codes, e4m3 block-16 scales) and fp8; it refuses int4
(``src/gen_worker/models/svdq.py:30-37``). This oracle keeps the reference's
*structure* step for step and swaps in the int4-g64 / int8 arithmetic:

* smoothing divide ``xs = x / smooth`` in fp32, rounded to bf16
  (``models/svdq_native.py:144``; fused form ``models/svdq_fused.py:88-92``);
* per-group absmax -> scale ``amax / (QMAX * s2)`` clamped and rounded to the
  stored scale dtype, then the codes divide by the *stored-precision* scale
  times ``s2`` (``models/nvfp4_quant.py:92-103``,
  ``models/svdq_fused.py:398-408``). int4: QMAX = 7, scale dtype fp16,
  group 64, codes ``clamp(rne(q), -8, 7)``;
* packing two codes per byte, element 2j in the LOW nibble
  (``models/nvfp4_quant.py:54-56``), two's-complement nibbles;
* int8 per-token activation quant = the reference's only int8 quantizer
  ``quantize_lowrank(scheme="int8")`` with the block = one row
  (``models/svdq_layout.py:261-275``); the W8A8 quantizer's per-tensor and
  static-scale modes (``models/w8a8.py:261-273``) with the same formula;
* GEMM + epilogue ``y = acc * (s2 * second) + la @ up^T + bias``
  (``models/svdq_fused.py:220-238``, ``:333-352``), with ``la = x @ proj_down``
  on RAW x (``models/svdq_fused.py:524``);
* the dense fallback ``W_eff = deq(W) / smooth + up @ down^T``
  (``models/svdq_native.py:200-221``).

Pinning (see tests/test_oracle.py): hand-computed known answers, exact
rational (``fractions``) brute force over bf16 patterns, integer brute force
for the group partial sums, torch's own bf16/fp16 conversions, and the
reference's structural tests (fold == two-branch, int8 round-trip bound).
"""

from __future__ import annotations

import numpy as np

GROUP = 64
INT4_QMAX = 7.0
INT4_MIN, INT4_MAX = -8, 7
FP16_MAX = 65504.0
SCALE_MIN_FP16 = 2.0 ** -24      # smallest positive fp16 (mirrors SCALE_MIN=2^-9, the smallest e4m3, models/nvfp4_quant.py:14)
INT8_QMAX = 127.0
INT8_SCALE_MIN = 1e-12           # models/svdq_layout.py:269


# ----------------------------------------------------------------------------
# bf16 / fp16 bit helpers (RNE, the rounding torch's .to(bfloat16) uses)
# ----------------------------------------------------------------------------

def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 array -> bf16 bit patterns (uint16), round-to-nearest-even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    bias = ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)
    r = ((u + bias) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(a: np.ndarray) -> np.ndarray:
    """float32 -> float32 holding the nearest bf16 value (RNE)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


# ----------------------------------------------------------------------------
# a1: smoothing divide
# ----------------------------------------------------------------------------

def smooth_divide(x_bits: np.ndarray, smooth_bits: np.ndarray | None) -> np.ndarray:
    """``xs = x2 / smooth_factor`` for bf16 tensors: fp32 divide, RNE to bf16.

    Follows ``models/svdq_native.py:144`` (torch bf16 division computes in
    fp32 and rounds once) and the fused form ``div_rn(x, sm).to(bfloat16)``
    in ``models/svdq_fused.py:88-92``. Returns bf16 bit patterns.
    """
    if smooth_bits is None:
        return np.ascontiguousarray(x_bits, dtype=np.uint16)
    x = bf16_bits_to_f32(x_bits)
    s = bf16_bits_to_f32(smooth_bits).reshape(1, -1)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        q = (x / s).astype(np.float32)
    return f32_to_bf16_bits(q)


# ----------------------------------------------------------------------------
# a3: int4 group-64 activation quantization
# ----------------------------------------------------------------------------

def int4_group_scale(amax: np.ndarray, s2: float = 1.0) -> np.ndarray:
    """Group absmax (fp32) -> fp16 scale.

    ``scale = clamp(amax / (QMAX * s2), SCALE_MIN, MAX)`` then cast to the
    stored dtype, exactly the order of ``models/nvfp4_quant.py:98-100`` with
    e4m3 replaced by fp16 and 6 by 7. The denominator ``QMAX * s2`` is an
    fp32 product as in ``models/svdq_fused.py:96``.
    """
    amax = np.asarray(amax, dtype=np.float32)
    den = np.float32(INT4_QMAX) * np.float32(s2)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        sc = (amax / den).astype(np.float32)
    sc = np.minimum(np.maximum(sc, np.float32(SCALE_MIN_FP16)), np.float32(FP16_MAX))
    return sc.astype(np.float16)


def quantize_int4_codes(xs_bits: np.ndarray, s2: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """bf16 smoothed activations [M, K] -> (int8 codes [M, K] in [-8, 7], fp16 scales [M, K/64]).

    Structure of ``quantize_activation_torch`` (``models/nvfp4_quant.py:96-102``):
    block view, ``amax`` over the block, scale in stored precision, then
    ``q = xb / (scale.float() * s2)`` (fp32 divide by the *rounded* scale),
    then the code cast. int4 code cast = ``round`` (RNE, as ``torch.round``
    in ``models/svdq_layout.py:272``) and clamp to [-8, 7].
    """
    m, k = xs_bits.shape
    if k % GROUP:
        raise ValueError(f"K={k} is not a multiple of the group size {GROUP}")
    xs = bf16_bits_to_f32(xs_bits).reshape(m, k // GROUP, GROUP)
    amax = np.abs(xs).max(axis=-1)
    sc = int4_group_scale(amax, s2)
    den = (sc.astype(np.float32) * np.float32(s2))[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = (xs / den).astype(np.float32)
    q = np.rint(q)
    q = np.clip(q, INT4_MIN, INT4_MAX).astype(np.int8)
    return q.reshape(m, k), sc


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """int codes [..., K] in [-8, 7] -> packed uint8 [..., K/2]; element 2j in the LOW nibble.

    Same byte convention as ``pack_e2m1`` (``models/nvfp4_quant.py:54-56``);
    nibbles are two's complement.
    """
    c = codes.astype(np.int16) & 0xF
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """packed uint8 [..., K/2] -> int8 codes [..., K] (two's complement nibbles)."""
    p = packed.astype(np.int16)
    lo = p & 0xF
    hi = (p >> 4) & 0xF
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.int16)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    out = np.where(out >= 8, out - 16, out)
    return out.astype(np.int8)


def quantize_act_int4(x_bits: np.ndarray, smooth_bits: np.ndarray | None = None,
                      s2: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """The ``svdq_quant`` op in int4 form: (packed uint8 [M, K/2], fp16 scales [M, K/64]).

    Mirrors ``_quant_smooth_kernel`` / ``_reference_quant_flat``
    (``models/svdq_fused.py:70-114``, ``:398-408``) with flat scales.
    """
    xs = smooth_divide(x_bits, smooth_bits)
    codes, sc = quantize_int4_codes(xs, s2)
    return pack_int4(codes), sc


def lowrank_down(x_bits: np.ndarray, proj_down_bits: np.ndarray) -> np.ndarray:
    """``la = x2 @ proj_down`` on RAW x (``models/svdq_fused.py:524``), in float64."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    d = bf16_bits_to_f32(proj_down_bits).astype(np.float64)
    return x @ d


# ----------------------------------------------------------------------------
# a5: group partial sums (exact integers)
# ----------------------------------------------------------------------------

def group_psums(qa_packed: np.ndarray, qw_packed: np.ndarray) -> np.ndarray:
    """int32 [M, N, G]: ``acc_g[m, n] = sum_{k in g} qx[m, k] * qw[n, k]``, exact."""
    qx = unpack_int4(qa_packed).astype(np.int64)
    qw = unpack_int4(qw_packed).astype(np.int64)
    m, k = qx.shape
    n = qw.shape[0]
    g = k // GROUP
    xg = qx.reshape(m, g, GROUP).transpose(1, 0, 2)    # [G, M, 64]
    wg = qw.reshape(n, g, GROUP).transpose(1, 2, 0)    # [G, 64, N]
    ps = np.matmul(xg, wg)                              # [G, M, N]
    return ps.transpose(1, 2, 0).astype(np.int32)


# ----------------------------------------------------------------------------
# a12: offline weight quantizers (producers)
# ----------------------------------------------------------------------------

def quantize_weight_int4(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp32 weight [N, K] -> (packed uint8 [N, K/2], fp16 scales [N, K/64]).

    Structure of ``quantize_nvfp4_tensor`` (``models/w4a4.py:140-154``):
    per-block absmax, ``bs[bs == 0] = 1``, clamp, cast to the stored scale
    dtype, divide by the stored scale, code cast. Single-level (no second
    scale), QMAX 7, fp16 scales, group 64.
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    blocks = w.reshape(n, k // GROUP, GROUP)
    bmax = np.abs(blocks).max(axis=-1)
    bs = (bmax / np.float32(INT4_QMAX)).astype(np.float32)
    bs[bs == 0] = 1.0
    bs = np.minimum(np.maximum(bs, np.float32(SCALE_MIN_FP16)), np.float32(FP16_MAX)).astype(np.float16)
    q = (blocks / bs.astype(np.float32)[..., None]).astype(np.float32)
    q = np.clip(np.rint(q), INT4_MIN, INT4_MAX).astype(np.int8).reshape(n, k)
    return pack_int4(q), bs


def dequantize_int4(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """(packed [R, K/2], fp16 scales [R, K/64]) -> float64 [R, K] (``dequantize_decoded`` form, ``models/svdq_layout.py:492-504``)."""
    q = unpack_int4(packed).astype(np.float64)
    r, k = q.shape
    s = scales.astype(np.float64).reshape(r, k // GROUP, 1)
    return (q.reshape(r, k // GROUP, GROUP) * s).reshape(r, k)


# ----------------------------------------------------------------------------
# W4A4 linear: the dequantize-then-matmul reference output
# ----------------------------------------------------------------------------

def w4a4_linear(x_bits: np.ndarray, smooth_bits: np.ndarray | None,
                qw: np.ndarray, sw: np.ndarray,
                proj_down_bits: np.ndarray | None, proj_up_bits: np.ndarray | None,
                bias_bits: np.ndarray | None, second: np.ndarray | None = None,
                s2: float = 1.0, gelu: bool = False) -> np.ndarray:
    """Full SVDQuant W4A4 linear in float64 (before the final output rounding).

    ``y = deq(qx) @ deq(qw)^T * (s2 * second) + (x @ down) @ up^T + bias``;
    activation quant as :func:`quantize_act_int4`. Structure of
    ``_SvdqLinear.forward`` (``models/svdq_native.py:140-156``) and the fused
    epilogue (``models/svdq_fused.py:220-238``). ``la`` is rounded to bf16
    like the reference's bf16 ``x2 @ proj_down``. ``gelu`` applies
    GELU-tanh after the bias (the fc1 -> GELU composition of config 2).
    """
    qa, sa = quantize_act_int4(x_bits, smooth_bits, s2)
    xd = dequantize_int4(qa, sa)
    wd = dequantize_int4(qw, sw)
    y = xd @ wd.T
    mult = np.float64(s2)
    if second is not None:
        y = y * (mult * np.asarray(second, dtype=np.float64).reshape(1, -1))
    elif s2 != 1.0:
        y = y * mult
    if proj_down_bits is not None and proj_up_bits is not None:
        la = lowrank_down(x_bits, proj_down_bits)
        la = bf16_bits_to_f32(f32_to_bf16_bits(la.astype(np.float32))).astype(np.float64)
        up = bf16_bits_to_f32(proj_up_bits).astype(np.float64)
        y = y + la @ up.T
    if bias_bits is not None:
        y = y + bf16_bits_to_f32(bias_bits).astype(np.float64).reshape(1, -1)
    if gelu:
        y = gelu_tanh(y)
    return y


def gelu_tanh(y: np.ndarray) -> np.ndarray:
    """GELU, tanh approximation (the Flux MLP activation)."""
    c = np.sqrt(2.0 / np.pi)
    return 0.5 * y * (1.0 + np.tanh(c * (y + 0.044715 * y ** 3)))


def fold_to_dense(qw: np.ndarray, sw: np.ndarray, smooth_bits: np.ndarray | None,
                  proj_down_bits: np.ndarray | None, proj_up_bits: np.ndarray | None) -> np.ndarray:
    """The any-hardware fallback weight ``W_eff = deq(W) / smooth + up @ down^T`` (``models/svdq_native.py:200-221``), float64 [N, K]."""
    w = dequantize_int4(qw, sw)
    if smooth_bits is not None:
        w = w / bf16_bits_to_f32(smooth_bits).astype(np.float64).reshape(1, -1)
    if proj_down_bits is not None and proj_up_bits is not None:
        up = bf16_bits_to_f32(proj_up_bits).astype(np.float64)
        down = bf16_bits_to_f32(proj_down_bits).astype(np.float64)
        w = w + up @ down.T
    return w


# ----------------------------------------------------------------------------
# a8 / a9: W8A8 int8
# ----------------------------------------------------------------------------

def quantize_act_int8(x_bits: np.ndarray, pertensor: bool = False,
                      static: float | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int8 activation quant: (codes int8 [M, K], fp32 scales [M, 1] or [1, 1]).

    ``quantize_lowrank(scheme="int8")`` (``models/svdq_layout.py:261-275``)
    with the block = one row: ``scale = (absmax / 127).clamp(min=1e-12)``,
    ``q = (x32 / scale).round().clamp(-127, 127)``. The reference W8A8
    quantizer's other modes (``models/w8a8.py:261-273``): ``pertensor`` takes
    the absmax over the whole tensor (scale [1, 1]); a ``static`` scale is
    used as given, [1, 1] if ``pertensor`` else repeated per row.
    """
    x = bf16_bits_to_f32(x_bits)
    m = x.shape[0]
    if static is not None:
        sa = np.full((1 if pertensor else m, 1), static, np.float32)
    else:
        amax = np.abs(x).max(axis=-1, keepdims=True).astype(np.float32)
        if pertensor:
            amax = amax.max(axis=0, keepdims=True)
        sa = np.maximum((amax / np.float32(INT8_QMAX)).astype(np.float32), np.float32(INT8_SCALE_MIN))
    with np.errstate(divide="ignore", invalid="ignore"):
        q = (x / sa).astype(np.float32)
    q = np.clip(np.rint(q), -INT8_QMAX, INT8_QMAX).astype(np.int8)
    return q, sa.astype(np.float32)


def quantize_weight_int8(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel int8 weights: (codes int8 [N, K], fp32 scales [N, 1]); same formula as :func:`quantize_act_int8` on fp32 rows (``models/svdq_layout.py:267-272``; scale shape ``[out, 1]`` of ``models/w8a8.py:341-342``)."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.abs(w).max(axis=-1, keepdims=True).astype(np.float32)
    sw = np.maximum((amax / np.float32(INT8_QMAX)).astype(np.float32), np.float32(INT8_SCALE_MIN))
    q = np.clip(np.rint((w / sw).astype(np.float32)), -INT8_QMAX, INT8_QMAX).astype(np.int8)
    return q, sw.astype(np.float32)


def int8_gemm(qa: np.ndarray, qw: np.ndarray) -> np.ndarray:
    """Exact int32 ``qa @ qw^T``."""
    return (qa.astype(np.int64) @ qw.astype(np.int64).T).astype(np.int32)


def w8a8_linear(x_bits: np.ndarray, qw: np.ndarray, sw: np.ndarray,
                bias: np.ndarray | None, pertensor: bool = False,
                static: float | None = None, ref_roundings: bool = False) -> np.ndarray:
    """``_scaled_mm(xq, W^T, scale_a=sa, scale_b=sw^T, bias)`` (``models/w8a8.py:374-378``) in float64,
    activation quant as :func:`quantize_act_int8`. The pertensor branch (``:366-372``) is the same product
    with every scale applied exactly, unless ``ref_roundings``: then it takes the reference's three bf16
    roundings, ``y0 = bf16(acc * sa)`` (``_scaled_mm`` with unit ``scale_b``, bf16 out), ``y1 = bf16(y0 *
    bf16(sw))`` (the weight scale cast to the output dtype), ``y = bf16(y1 + bias)`` (a bf16 bias), returned
    as float64 values of those bf16 numbers."""
    qa, sa = quantize_act_int8(x_bits, pertensor, static)
    acc = int8_gemm(qa, qw).astype(np.float64)
    if ref_roundings and pertensor:
        y0 = round_bf16((acc * sa.astype(np.float64)).astype(np.float32))
        sw16 = round_bf16(sw.astype(np.float32).reshape(1, -1))
        y = round_bf16((y0.astype(np.float64) * sw16.astype(np.float64)).astype(np.float32))
        if bias is not None:
            b16 = round_bf16(np.asarray(bias, dtype=np.float32).reshape(1, -1))
            y = round_bf16((y.astype(np.float64) + b16.astype(np.float64)).astype(np.float32))
        return y.astype(np.float64)
    y = acc * sa.astype(np.float64) * sw.astype(np.float64).reshape(1, -1)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64).reshape(1, -1)
    return y


# ----------------------------------------------------------------------------
# acceptance metrics
# ----------------------------------------------------------------------------

def max_abs_err(y: np.ndarray, ref: np.ndarray) -> float:
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref))) if ref.size else 0.0


def mean_rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """mean |y - ref| / mean |ref| (the mean relative error of the whole output)."""
    if ref.size == 0:
        return 0.0
    den = float(np.mean(np.abs(ref)))
    return float(np.mean(np.abs(np.asarray(y, np.float64) - ref))) / max(den, 1e-30)
