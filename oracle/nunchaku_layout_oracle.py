"""CPU oracle for the nunchaku svdq int4 checkpoint layout.

TEST INFRASTRUCTURE ONLY (only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it, as the checker).

It restates deepcompressor's forward packers -- the ones the reference's own
tests restate to pin its decoders (``tests/test_svdq_official_layout_pgw770.py:
31-96``: ``pack_weight`` bits=4, ``pack_scale``, ``pack_lowrank_weight``) --
as explicit index arithmetic, one element at a time, so they cross-check the
product's tensor reshapes:

* weight: code (n, k) with n = 128 nt + 16 np + 8 ns + nl and
  k = 64 kt + 32 ks + 8 kl + kr goes to nibble kr of int32 word
  ((((((nt * KT + kt) * 8 + np) * 8 + nl) * 4 + kl) * 2 + ns) * 2 + ks)
  (the reference's permutation (0, 5, 6, 1, 3, 8, 2, 7, 4, 9),
  ``models/svdq_layout.py:14-15``);
* scale grid [n, G] (G = 1: a vector): row n = 128 b + 16 a + 8 p + 2 c + d,
  group g goes to flat position (b * G + g) * 128 + 16 a + 4 c + 2 p + d
  (``pack_scale``'s reshape (n/128, 1, 8, 2, 4, 2, G) and permutation
  (0, 6, 1, 2, 4, 3, 5), the reference's ``_VEC_*`` constants,
  ``models/svdq_layout.py:24-25``);
* low-rank factor, 16 x 16 packs: element (i_n, i_k) of pack (cp, rp), with
  i_n = 8 ns + nl and i_k = 8 ks + 2 kl + kr, goes to flat position
  ((((((cp * RP + rp) * 8 + nl) * 4 + kl) * 2 + ns) * 2 + ks) * 2 + kr)
  (``models/svdq_layout.py:27-31``); for proj_down i_n runs over the rank
  and i_k over the input, for proj_up i_n over the output and i_k over the
  rank;
* fp4 micro-scales (``pack_micro_scale``, the reference test's restatement at
  ``tests/test_svdq_official_layout_pgw770.py:47-63``, decoded by
  ``models/svdq_layout.py:110-125``): scale [n, NB] (one e4m3 per 16 inputs),
  row n = 128 t + 32 a + 8 b + c and block = 4 q + j, goes to flat position
  ((((t * Q + q) * 8 + c) * 4 + b) * 4 + a) * 4 + j of the stored [NB, n]
  grid (Q = NB / 4), the (4, 4, 8) row split with the lane index c
  outermost.
"""

from __future__ import annotations

import numpy as np


def pack_weight(codes: np.ndarray) -> np.ndarray:
    """nibble codes uint8 [n, k] -> qweight int8 [n, k/2]."""
    n, k = codes.shape
    kt_n = k // 64
    words = np.zeros(n * k // 8, dtype=np.uint32)
    for row in range(n):
        nt, r = divmod(row, 128)
        np_, r = divmod(r, 16)
        ns, nl = divmod(r, 8)
        for col in range(k):
            kt, c = divmod(col, 64)
            ks, c = divmod(c, 32)
            kl, kr = divmod(c, 8)
            w = (((((nt * kt_n + kt) * 8 + np_) * 8 + nl) * 4 + kl) * 2 + ns) * 2 + ks
            words[w] |= np.uint32(int(codes[row, col]) & 0xF) << np.uint32(4 * kr)
    return words.view(np.int8).reshape(n, k // 2)


def pack_scale(scales: np.ndarray) -> np.ndarray:
    """[n, G] -> stored grid [G, n] (flat memory in the packed order)."""
    n, g_n = scales.shape
    flat = np.zeros(n * g_n, dtype=scales.dtype)
    for row in range(n):
        b, r = divmod(row, 128)
        a, r = divmod(r, 16)
        p, r = divmod(r, 8)
        c, d = divmod(r, 2)
        for g in range(g_n):
            flat[(b * g_n + g) * 128 + 16 * a + 4 * c + 2 * p + d] = scales[row, g]
    return flat.reshape(g_n, n)


def pack_lowrank(weight: np.ndarray, *, down: bool) -> np.ndarray:
    """Logical [in, rank] (down) / [out, rank] (up) -> the stored tensor (same shape)."""
    c_n, r_n = weight.shape
    rp_n = r_n // 16
    flat = np.zeros(c_n * r_n, dtype=weight.dtype)
    for row in range(c_n):
        for col in range(r_n):
            cp, ic = divmod(row, 16)
            rp, ir = divmod(col, 16)
            i_n, i_k = (ir, ic) if down else (ic, ir)
            ns, nl = divmod(i_n, 8)
            ks, rem = divmod(i_k, 8)
            kl, kr = divmod(rem, 2)
            f = (((((cp * rp_n + rp) * 8 + nl) * 4 + kl) * 2 + ns) * 2 + ks) * 2 + kr
            flat[f] = weight[row, col]
    return flat.reshape(c_n, r_n)


def pack_micro_scale(scales: np.ndarray) -> np.ndarray:
    """e4m3 scale bytes [n, NB] -> the stored grid [NB, n]."""
    n, nb = scales.shape
    q_n = nb // 4
    flat = np.zeros(n * nb, dtype=scales.dtype)
    for row in range(n):
        t, r = divmod(row, 128)
        a, r = divmod(r, 32)
        b, c = divmod(r, 8)
        for blk in range(nb):
            q, j = divmod(blk, 4)
            flat[((((t * q_n + q) * 8 + c) * 4 + b) * 4 + a) * 4 + j] = scales[row, blk]
    return flat.reshape(nb, n)
