"""CPU oracle for the nvfp4 compatibility lane.

TEST INFRASTRUCTURE ONLY (only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it, as the checker).

Restates, in numpy float32 arithmetic (IEEE division and rounding, like the
reference's torch ops on fp32 tensors):

* ``e4m3_rne``: fp32 -> float8_e4m3fn bits, round to nearest even (the
  ``.to(torch.float8_e4m3fn)`` of ``models/nvfp4_quant.py:99`` and
  ``models/w4a4.py:150``), by exponent/mantissa arithmetic; ``e4m3_value``
  decodes;
* ``cast_e2m1`` (``models/nvfp4_quant.py:41-51``): bounds
  {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0}, ties at 0.75, 1.75, 2.5 bumped up;
* ``pack_e2m1`` / ``unpack_e2m1`` (``:54-69``);
* ``to_blocked_scales`` (``:72-84``) as an explicit index loop;
* ``quantize_activation`` = ``quantize_activation_torch`` (``:92-103``);
* ``quantize_nvfp4_tensor`` / ``dequantize_nvfp4_tensor``
  (``models/w4a4.py:140-164``), including the weight quantizer's
  zero-block rule ``bs[bs == 0] = 1.0``;
* ``nvfp4_linear`` = ``_W4A4Linear.forward`` (``models/w4a4.py:336-352``):
  the fp4 product summed in float64 and rounded to bf16 (torch._scaled_mm
  with a bf16 out_dtype), times bf16(s2 * weight_scale_2), plus the bf16 bias;
* ``svdq_fp4_linear`` = the svdq fp4 module's forward (``_SvdqLinear.forward``,
  ``models/svdq_native.py:140-156``): the activation divided by the smoothing
  factors (bf16), the dynamic scale s2 = max|xs| / (6 * 448), the fp4 product
  rounded to bf16, times bf16(s2 * second) (second per output channel or per
  tensor), plus the low-rank branch on the RAW activation
  bf16(bf16(x @ down) @ up^T), plus the bias, each sum rounded to bf16.
"""

from __future__ import annotations

import numpy as np

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)
BOUNDS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
SCALE_MIN, FP8_MAX, E2M1_MAX = np.float32(2.0 ** -9), np.float32(448.0), np.float32(6.0)


E4M3_NAN = 0x7F   # float8_e4m3fn has no infinity; S.1111.111 is NaN


def e4m3_value(code) -> np.ndarray:
    """float8_e4m3fn bits (sign bit ignored) -> float32; 0x7F is NaN."""
    c = np.asarray(code, np.int64) & 0x7F
    e, m = c >> 3, c & 7
    with np.errstate(invalid="ignore"):
        v = np.where(e == 0, m / 512.0, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    return np.where(c == E4M3_NAN, np.nan, v).astype(np.float32)


def e4m3_rne(v) -> np.ndarray:
    """fp32 in [2^-9, 448] -> e4m3fn bits, nearest value, ties to the even code; NaN -> 0x7F (torch's
    ``.to(torch.float8_e4m3fn)`` of a NaN, what the reference's clamp passes through)."""
    v = np.asarray(v, np.float32)
    u = v.view(np.uint32).astype(np.int64)
    e = (u >> 23) - 127
    m = u & 0x7FFFFF
    r = m >> 20
    rem = m & 0xFFFFF
    up = (rem > 0x80000) | ((rem == 0x80000) & ((r & 1) == 1))
    normal = ((e + 7) << 3) + r + up
    with np.errstate(invalid="ignore"):
        sub = np.rint(np.nan_to_num(v.astype(np.float64)) * 512.0).astype(np.int64)  # exact; ties to even
    out = np.where(e < -6, sub, normal)
    return np.where(np.isnan(v), E4M3_NAN, out).astype(np.uint8)


def cast_e2m1(q) -> np.ndarray:
    """``cast_e2m1``: the count of bounds below |q| (``searchsorted``), tie bumps, sign from q < 0; a NaN
    sorts after every bound (code 7, sign clear: NaN < 0 is false)."""
    q = np.asarray(q, np.float32)
    a = np.abs(q)
    c = np.zeros(q.shape, np.int64)
    for b in BOUNDS:
        c += a > b
    c += (a == 0.75) | (a == 1.75) | (a == 2.5)
    c = np.where(np.isnan(a), len(BOUNDS), c)
    return (c + 8 * (q < 0)).astype(np.uint8)


def dynamic_s2(x: np.ndarray) -> np.float32:
    """The forward's dynamic second-level scale (``models/w4a4.py:342-343``): max(max|x| / 2688, 1e-12);
    a NaN anywhere makes it NaN (torch's amax and clamp propagate NaN)."""
    amax = np.float32(np.abs(np.asarray(x, np.float32)).max())
    return np.float32(np.maximum(np.float32(amax / np.float32(2688.0)), np.float32(1e-12)))


def pack_e2m1(codes: np.ndarray) -> np.ndarray:
    return ((codes[..., 1::2] << 4) | codes[..., 0::2]).astype(np.uint8)


def unpack_e2m1(packed: np.ndarray) -> np.ndarray:
    lut = np.concatenate([E2M1, -E2M1])
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), np.float32)
    out[..., 0::2] = lut[packed & 0xF]
    out[..., 1::2] = lut[packed >> 4]
    return out


def blocked_scale_numel(rows: int, kb: int) -> int:
    return (rows + 127) // 128 * 128 * ((kb + 3) // 4) * 4


def to_blocked_scales(flat: np.ndarray) -> np.ndarray:
    """[rows, kb] scale bytes -> the blocked order, zero padded, one element at a time."""
    rows, kb = flat.shape
    ncb = (kb + 3) // 4
    out = np.zeros(blocked_scale_numel(rows, kb), np.uint8)
    for r in range(rows):
        for c in range(kb):
            tile = (r // 128) * ncb + c // 4
            out[tile * 512 + (r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4] = flat[r, c]
    return out


def from_blocked_scales(blocked: np.ndarray, rows: int, kb: int) -> np.ndarray:
    ncb = (kb + 3) // 4
    r = np.arange(rows)[:, None]
    c = np.arange(kb)[None, :]
    idx = ((r // 128) * ncb + c // 4) * 512 + (r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4
    return blocked[idx]


def quantize_activation(x: np.ndarray, s2: float) -> tuple[np.ndarray, np.ndarray]:
    """float32 [M, K] (bf16 values) + s2 -> (packed codes [M, K/2], flat e4m3 scale bytes [M, K/16])."""
    m, k = x.shape
    xb = x.astype(np.float32).reshape(m, k // 16, 16)
    s2 = np.float32(s2)
    bmax = np.abs(xb).max(axis=-1)
    t = np.clip(bmax / (E2M1_MAX * s2), SCALE_MIN, FP8_MAX).astype(np.float32)
    sc = e4m3_rne(t)
    den = (e4m3_value(sc) * s2).astype(np.float32)
    q = (xb / den[..., None]).astype(np.float32)
    return pack_e2m1(cast_e2m1(q.reshape(m, k))), sc


def dequantize(packed: np.ndarray, scales_flat: np.ndarray, s2: float = 1.0) -> np.ndarray:
    """codes + flat scale bytes (+ the second-level scale) -> float32 [rows, K]."""
    vals = unpack_e2m1(packed)
    rows, k = vals.shape
    return (vals.reshape(rows, k // 16, 16) * e4m3_value(scales_flat)[..., None]
            * np.float32(s2)).reshape(rows, k).astype(np.float32)


def quantize_nvfp4_tensor(w: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.float32]:
    """The offline weight quantizer: (packed [out, in/2], flat e4m3 scale bytes [out, in/16], ws2)."""
    wf = w.astype(np.float32)
    n, k = wf.shape
    ws2 = np.float32(max(np.float32(np.abs(wf).max()) / np.float32(E2M1_MAX * FP8_MAX), np.float32(1e-12)))
    blocks = wf.reshape(n, k // 16, 16)
    bs = (np.abs(blocks).max(axis=-1) / (E2M1_MAX * ws2)).astype(np.float32)
    bs[bs == 0] = 1.0
    sc = e4m3_rne(np.clip(bs, SCALE_MIN, FP8_MAX).astype(np.float32))
    q = (blocks / (e4m3_value(sc) * ws2)[..., None]).astype(np.float32)
    return pack_e2m1(cast_e2m1(q.reshape(n, k))), sc, ws2


def bf16_round(a) -> np.ndarray:
    """float -> the nearest bf16 value (ties to even), as float32."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def nvfp4_linear(x: np.ndarray, s2: float, wq: np.ndarray, ws_flat: np.ndarray, ws2: float,
                 bias=None) -> np.ndarray:
    """The module forward on bf16-valued float32 inputs: float64 [M, N] (the bf16 values of the result)."""
    xq, xs = quantize_activation(x, s2)
    acc = dequantize(xq, xs).astype(np.float64) @ dequantize(wq, ws_flat).astype(np.float64).T
    y = bf16_round(acc.astype(np.float32))
    y = bf16_round(y * bf16_round(np.float32(s2) * np.float32(ws2)))
    if bias is not None:
        y = bf16_round(y + np.asarray(bias, np.float32))
    return y.astype(np.float64)


def svdq_fp4_linear(x: np.ndarray, smooth, wq: np.ndarray, ws_flat: np.ndarray, second, down=None, up=None,
                    bias=None, s2=None) -> np.ndarray:
    """bf16-valued float32 x [M, K]; smooth [K] or None; packed codes wq [N, K/2]; flat e4m3 scale bytes
    ws_flat [N, K/16]; second [N] or [1]; down [K, r] and up [N, r] or None; bias [N] or None; s2 the call's
    dynamic scale (computed from x when None; a row sample passes the full call's) -> float64 [M, N]."""
    x = np.asarray(x, np.float32)
    xs = x if smooth is None else bf16_round(x / np.asarray(smooth, np.float32).reshape(1, -1))
    s2 = dynamic_s2(xs) if s2 is None else np.float32(s2)
    xq, xsc = quantize_activation(xs, s2)
    acc = dequantize(xq, xsc).astype(np.float64) @ dequantize(wq, ws_flat).astype(np.float64).T
    y = bf16_round(acc.astype(np.float32))
    y = bf16_round(y * bf16_round(np.float32(s2) * np.asarray(second, np.float32).reshape(1, -1)))
    if down is not None:
        t = bf16_round((x.astype(np.float64) @ np.asarray(down, np.float64)).astype(np.float32))
        lr = bf16_round((t.astype(np.float64) @ np.asarray(up, np.float64).T).astype(np.float32))
        y = bf16_round(y + lr)
    if bias is not None:
        y = bf16_round(y + np.asarray(bias, np.float32).reshape(1, -1))
    return y.astype(np.float64)
