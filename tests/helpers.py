"""Shared test helpers: bit views and the output tolerance of the north star."""

from __future__ import annotations

import numpy as np
import torch

from oracle import svdq_oracle as O

# Output acceptance vs the float64 dequantize-then-matmul reference:
#   max-abs error <= 2e-2 beyond the output dtype's own rounding (half an ulp of
#   the reference value, 2^-8 |ref| for bf16 and 2^-11 |ref| for fp16), and
#   mean relative error (mean|y - ref| / mean|ref|) <= 5e-3.
MAX_ABS = 2e-2
MEAN_REL = 5e-3
REL_FRO = 2e-2   # the reference's own GEMM gate (models/w4a4.py:201-202)


def bits16(t: torch.Tensor) -> np.ndarray:
    """16-bit tensor (bf16/fp16) -> numpy uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, dtype: torch.dtype, device="cpu") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype).to(device)


def check_output(y: torch.Tensor, ref: np.ndarray, *, what: str = "") -> dict:
    yf = y.detach().float().cpu().numpy().astype(np.float64)
    ulp_rel = 2.0 ** -8 if y.dtype == torch.bfloat16 else 2.0 ** -11
    err = np.abs(yf - ref)
    excess = float(np.max(err - ulp_rel * np.abs(ref))) if ref.size else 0.0
    stats = {
        "max_abs": O.max_abs_err(yf, ref),
        "max_abs_beyond_rounding": excess,
        "mean_rel": O.mean_rel_err(yf, ref),
        "rel_fro": float(np.linalg.norm(yf - ref) / max(np.linalg.norm(ref), 1e-30)) if ref.size else 0.0,
    }
    # the plain max-abs error is printed beside the relaxed bound (bf16 outputs above ~5 carry a half-ulp
    # rounding larger than 2e-2 by themselves)
    print(f"{what}: max_abs {stats['max_abs']:.3e} (beyond the output rounding {excess:.3e}), mean_rel "
          f"{stats['mean_rel']:.3e}, rel_fro {stats['rel_fro']:.3e}")
    assert np.isfinite(yf).all(), f"{what}: non-finite output"
    assert excess <= MAX_ABS, f"{what}: {stats}"
    assert stats["mean_rel"] <= MEAN_REL, f"{what}: {stats}"
    assert stats["rel_fro"] <= REL_FRO, f"{what}: {stats}"
    return stats


# e3m2 fp6 (sign, 3-bit exponent with bias 3, 2-bit mantissa): the integers -8 .. 8 it holds
_E3M2_INT = {0x00: 0, 0x0C: 1, 0x10: 2, 0x12: 3, 0x14: 4, 0x15: 5, 0x16: 6, 0x17: 7, 0x18: 8}


def decode_fp6_codes(q6: np.ndarray) -> np.ndarray:
    """uint8 [M, 3K/4] (element t of each group at bits [6t, 6t+6) of its 48 bytes, little-endian)
    -> int8 codes [M, K]; raises on any 6-bit value that is not an integer in [-8, 8]."""
    q6 = np.asarray(q6, np.uint8)
    m, nb = q6.shape
    k = nb * 4 // 3
    b = q6.reshape(m, k // 4, 3).astype(np.uint32)
    word = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16)               # 4 codes per 3 bytes
    codes = np.stack([(word >> (6 * t)) & 0x3F for t in range(4)], axis=-1).reshape(m, k)
    mag = codes & 0x1F
    lut = np.full(32, 127, np.int64)
    for bits, val in _E3M2_INT.items():
        lut[bits] = val
    v = lut[mag]
    if np.any(v == 127):
        raise AssertionError(f"non-integer e3m2 code(s): {sorted(set(int(c) for c in codes[v == 127].ravel()))[:8]}")
    return np.where(codes & 0x20, -v, v).astype(np.int8)


FP6_REC = 104


def decode_fp6_records(rec: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp6 operand records uint8 [K/128, M, 104] (per 128-column stage and row: 96 bytes of e3m2 codes,
    then the stage's two fp16 group scales) -> (int8 codes [M, K], fp16 scale bits uint16 [M, K/64])."""
    rec = np.asarray(rec, np.uint8)
    s, m, width = rec.shape
    assert width == FP6_REC, rec.shape
    codes = decode_fp6_codes(rec[:, :, :96].transpose(1, 0, 2).reshape(m, s * 96))
    scales = rec[:, :, 96:100].copy().view(np.uint16).transpose(1, 0, 2).reshape(m, 2 * s)
    return codes, scales
