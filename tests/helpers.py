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
    assert np.isfinite(yf).all(), f"{what}: non-finite output"
    assert excess <= MAX_ABS, f"{what}: {stats}"
    assert stats["mean_rel"] <= MEAN_REL, f"{what}: {stats}"
    assert stats["rel_fro"] <= REL_FRO, f"{what}: {stats}"
    return stats
