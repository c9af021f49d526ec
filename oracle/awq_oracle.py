"""CPU oracle for the AWQ W4A16 modulation lane.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker. The product (``gen_worker_amd``) never imports it.

What this restates (numpy, explicit index arithmetic rather than the
product's tensor reshapes, so the two cross-check):

* the TinyChat nibble interleave of the on-disk ``qweight``
  (``src/gen_worker/models/svdq_awq.py:31-46`` unpack, ``:140-151`` pack):
  per row, 32-code block b -> 8 16-bit words, word j = codes 32b + j, +8,
  +16, +24 in nibbles 0..3; rows interleaved in groups of 4 per 64 columns;
* the padded scale-grid row count ``num_scale_rows`` (``:18-28``);
* the dequantized weight w = code * scale + zero in fp32, rounded to bf16
  where the lane holds bf16 weights (``:74-82`` and the bf16 copy of
  ``decode_awq_linear``, ``:106-129``; the packed kernel's
  ``(q * s + z).to(bf16)``, ``models/svdq_awq_packed.py:84-89``);
* y = x @ w^T + bias (``models/svdq_awq_packed.py:90-94``), here in float64;
* the exporter's adaLN transform and its inverse (``models/svdq_awq.py:85-103``,
  ``:154-171``).

Pinning (tests/test_awq.py): a one-hot placement table for the interleave
derived from the word/row positions, exact rational arithmetic for the
dequantized bf16 values, hand-computed adaLN permutations and bias offsets,
and the scale-row counts for the shapes Flux uses.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np

from .svdq_oracle import bf16_bits_to_f32, f32_to_bf16_bits


def num_scale_rows(ic: int, gs: int) -> int:
    groups = ic // gs
    packs = (groups + 7) // 8
    mult = {32: 4, 64: 2}.get(gs, 1)
    packs = (packs + mult - 1) // mult * mult
    return packs * 8


def tinychat_pack(codes: np.ndarray) -> np.ndarray:
    """codes uint8 [oc, ic] (0..15) -> int32 [oc/4, ic/2], one word at a time."""
    oc, ic = codes.shape
    words = np.zeros((oc // 4, ic), dtype=np.uint16)
    for r in range(oc):
        for b in range(ic // 32):
            for j in range(8):
                w = 0
                for nib in range(4):
                    w |= int(codes[r, 32 * b + 8 * nib + j]) << (4 * nib)
                wi = 8 * b + j                       # word index within row r
                c64, u = divmod(wi, 16)             # 64-column unit, word within it
                words[r // 4, 64 * c64 + 16 * (r % 4) + u] = w
    return words.view(np.int16).view(np.int32).reshape(oc // 4, ic // 2)


def tinychat_unpack(packed: np.ndarray, oc: int, ic: int) -> np.ndarray:
    words = np.ascontiguousarray(packed).view(np.uint16).reshape(oc // 4, ic)
    codes = np.zeros((oc, ic), dtype=np.uint8)
    for r in range(oc):
        for wi in range(ic // 4):
            c64, u = divmod(wi, 16)
            w = int(words[r // 4, 64 * c64 + 16 * (r % 4) + u])
            b, j = divmod(wi, 8)
            for nib in range(4):
                codes[r, 32 * b + 8 * nib + j] = (w >> (4 * nib)) & 0xF
    return codes


def dequant_f32(codes: np.ndarray, scale_bits: np.ndarray, zero_bits: np.ndarray) -> np.ndarray:
    """codes [oc, ic]; scale / zero bf16 bits [oc, ic/64] -> fp32 code * s + z (two fp32 roundings, the
    product exact)."""
    oc, ic = codes.shape
    s = np.repeat(bf16_bits_to_f32(scale_bits), 64, axis=1)
    z = np.repeat(bf16_bits_to_f32(zero_bits), 64, axis=1)
    return (codes.astype(np.float32) * s).astype(np.float32) + z


def dequant_bf16_bits(codes: np.ndarray, scale_bits: np.ndarray, zero_bits: np.ndarray) -> np.ndarray:
    """The bf16 weight the packed lane multiplies by (bits, uint16 [oc, ic])."""
    return f32_to_bf16_bits(dequant_f32(codes, scale_bits, zero_bits))


def dequant_exact_bf16_bits(code: int, scale_bits: int, zero_bits: int) -> int:
    """One element by exact rational arithmetic: RN_f32(code * s + z) then RN_bf16 (both ties to even)."""
    s = Fraction(float(bf16_bits_to_f32(np.array([scale_bits], np.uint16))[0]))
    z = Fraction(float(bf16_bits_to_f32(np.array([zero_bits], np.uint16))[0]))
    v = code * s + z
    f32 = _round_fraction(v, 24)
    return int(f32_to_bf16_bits(np.array([float(f32)], np.float32))[0])


def _round_fraction(v: Fraction, bits: int) -> Fraction:
    """Round a rational to the nearest binary float with a ``bits``-bit significand, ties to even (normal
    range; the tests keep values normal)."""
    if v == 0:
        return v
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = 0
    while a >= 2:
        a /= 2
        e += 1
    while a < 1:
        a *= 2
        e -= 1
    scaled = a * (1 << (bits - 1))
    fl = scaled.numerator // scaled.denominator
    rem = scaled - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * Fraction(fl, 1 << (bits - 1)) * (Fraction(2) ** e)


def awq_linear(x_bits: np.ndarray, codes: np.ndarray, scale_bits: np.ndarray, zero_bits: np.ndarray,
               bias_bits: np.ndarray | None) -> np.ndarray:
    """float64 y [M, N] = x @ w_bf16^T + bias (bias bf16)."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = bf16_bits_to_f32(dequant_bf16_bits(codes, scale_bits, zero_bits)).astype(np.float64)
    y = x @ w.T
    if bias_bits is not None:
        y = y + bf16_bits_to_f32(bias_bits).astype(np.float64)[None, :]
    return y


def adanorm_apply(w: np.ndarray, b: np.ndarray, splits: int) -> tuple[np.ndarray, np.ndarray]:
    """Stored row j*splits + s <- original row s*per + j; bias of splits 1 and splits-2 += 1."""
    oc = w.shape[0]
    per = oc // splits
    wo = np.empty_like(w)
    bo = np.empty(oc, dtype=np.float64)
    for s in range(splits):
        for j in range(per):
            wo[j * splits + s] = w[s * per + j]
            bo[j * splits + s] = float(b[s * per + j]) + (1.0 if s in (1, splits - 2) else 0.0)
    return wo, bo


def adanorm_undo(w: np.ndarray, b: np.ndarray, splits: int) -> tuple[np.ndarray, np.ndarray]:
    oc = w.shape[0]
    per = oc // splits
    wo = np.empty_like(w)
    bo = np.empty(oc, dtype=np.float64)
    for s in range(splits):
        for j in range(per):
            wo[s * per + j] = w[j * splits + s]
            bo[s * per + j] = float(b[j * splits + s]) - (1.0 if s in (1, splits - 2) else 0.0)
    return wo, bo
