"""Pins the CPU oracle (oracle/svdq_oracle.py) before anything is checked against it.

Each check is independent of the oracle's own code path: hand-computed known
answers, exact rational arithmetic (``fractions``), integer brute force, torch's
own bf16/fp16 conversions, and the reference's structural tests
(fold == two-branch, int8 round-trip bound). The reference holds no numeric
golden vectors for this path (its lane is nvfp4 and it refuses int4,
src/gen_worker/models/svdq.py:30-37).
"""

from __future__ import annotations

import struct
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import svdq_oracle as O


# ---------------------------------------------------------------------------
# exact-arithmetic helpers (independent of numpy's float paths)
# ---------------------------------------------------------------------------

def _f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def _round_to_format(q: Fraction, mant_bits: int, emin: int) -> Fraction:
    """Round a positive rational to the nearest binary float with `mant_bits` significand bits
    (incl. implicit) and minimum normal exponent `emin`, ties to even. No overflow handling."""
    if q == 0:
        return Fraction(0)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - (mant_bits - 1))
    n = q / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl * ulp


def _rn_f32(q: Fraction) -> Fraction:
    s = -1 if q < 0 else 1
    return s * _round_to_format(abs(q), 24, -126)


def _rn_f16(q: Fraction) -> Fraction:
    s = -1 if q < 0 else 1
    return s * _round_to_format(abs(q), 11, -14)


def _rne_int(q: Fraction) -> int:
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def _bf16_bits(v: float) -> int:
    return int(O.f32_to_bf16_bits(np.array([v], np.float32))[0])


# ---------------------------------------------------------------------------
# number formats vs torch
# ---------------------------------------------------------------------------

def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(11)
    a = torch.randn(200_000, generator=g) * torch.exp(torch.randn(200_000, generator=g) * 8)
    specials = torch.tensor([0.0, -0.0, 1.0, 1.00390625, 1.0078125 + 2 ** -9, 3.3895313892515355e38,
                             1e-40, -1e-41, float("inf"), -float("inf")])
    a = torch.cat([a, specials])
    want = a.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16_bits(a.numpy())
    assert np.array_equal(got, want)


def test_fp16_scale_rounding_matches_torch():
    g = torch.Generator().manual_seed(12)
    a = (torch.rand(100_000, generator=g) * 30).float()
    a = torch.cat([a, torch.tensor([0.0, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 65504.0, 65519.0])])
    want = a.to(torch.float16).numpy()
    got = a.numpy().astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_smooth_divide_matches_torch_bf16_division():
    g = torch.Generator().manual_seed(13)
    x = torch.randn(64, 512, generator=g).to(torch.bfloat16)
    sm = (torch.rand(512, generator=g) * 3.75 + 0.25).to(torch.bfloat16)
    want = (x / sm).view(torch.int16).numpy().view(np.uint16)
    got = O.smooth_divide(x.view(torch.int16).numpy().view(np.uint16), sm.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(got, want)


def test_smooth_divide_exact_rational_all_bf16():
    """Every finite bf16 x divided by a fixed awkward bf16 divisor == RN_bf16(RN_f32(x/s)) exactly."""
    bits = np.arange(0, 0x7F80, 7, dtype=np.uint16)  # positive finite bf16, strided sample
    s_bits = _bf16_bits(1.7109375)  # 0x3FDB -> 1.7109375
    xs = O.smooth_divide(bits.reshape(1, -1), np.full(bits.shape, s_bits, np.uint16))[0]
    s = Fraction(_f32(s_bits << 16))
    for b, got in zip(bits.tolist(), xs.tolist()):
        q = _rn_f32(Fraction(_f32(b << 16)) / s)
        want = _round_to_format(q, 8, -126) if q else Fraction(0)
        assert Fraction(_f32(got << 16)) == want, hex(b)


# ---------------------------------------------------------------------------
# int4 group quantization
# ---------------------------------------------------------------------------

def _group(vals):
    g = np.zeros(64, np.float32)
    g[: len(vals)] = vals
    return O.f32_to_bf16_bits(g).reshape(1, 64)


def test_int4_known_answers():
    # amax = 7 -> scale exactly 1.0; RNE ties 2.5->2, -2.5->-2, 1.5->2, 0.5->0, -3.5->-4
    codes, sc = O.quantize_int4_codes(_group([7.0, -7.0, 2.5, -2.5, 1.5, 0.5, -3.5, 6.5, 4.0]))
    assert float(sc[0, 0]) == 1.0
    assert codes[0, :9].tolist() == [7, -7, 2, -2, 2, 0, -4, 6, 4]
    assert not codes[0, 9:].any()
    # amax = 3.5 -> scale 0.5
    codes, sc = O.quantize_int4_codes(_group([3.5, 1.25, -0.75, 0.25]))
    assert float(sc[0, 0]) == 0.5
    assert codes[0, :4].tolist() == [7, 2, -2, 0]
    # zero group -> smallest positive fp16 scale, all-zero codes
    codes, sc = O.quantize_int4_codes(np.zeros((1, 64), np.uint16))
    assert sc.view(np.uint16)[0, 0] == 0x0001 and not codes.any()
    # s2 (second-level scale) divides the scale: amax 7, s2 2 -> scale 0.5, codes q = x / (0.5 * 2)
    codes, sc = O.quantize_int4_codes(_group([7.0, 3.0]), s2=2.0)
    assert float(sc[0, 0]) == 0.5 and codes[0, :2].tolist() == [7, 3]


def test_int4_scale_exact_rational_all_amax():
    """scale = RN_f16(clamp(RN_f32(amax / 7))) for a sweep of bf16 amax values."""
    bits = np.arange(1, 0x7F80, 13, dtype=np.uint16)
    amax = O.bf16_bits_to_f32(bits)
    got = O.int4_group_scale(amax).astype(np.float64)
    for b, g in zip(bits.tolist(), got.tolist()):
        a = Fraction(_f32(b << 16))
        q = _rn_f32(a / 7)
        q = min(max(q, Fraction(2) ** -24), Fraction(65504))
        want = _rn_f16(q)
        assert Fraction(g) == want, hex(b)


def test_int4_codes_exact_rational_brute_force():
    """Every bf16 value v in [-amax, amax] in a group whose scale is an awkward fp16:
    code == clamp(rne(RN_f32(v / scale)), -8, 7), computed with exact rationals."""
    amax = 5.1875  # bf16-exact
    all_bits = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    vals = O.bf16_bits_to_f32(all_bits)
    ok = np.isfinite(vals) & (np.abs(vals) <= amax)
    vals = vals[ok][::3]
    n = vals.size
    pad = (-n) % 63
    vals = np.concatenate([vals, np.zeros(pad, np.float32)])
    rows = vals.reshape(-1, 63)
    grid = np.concatenate([np.full((rows.shape[0], 1), amax, np.float32), rows], axis=1)
    codes, sc = O.quantize_int4_codes(O.f32_to_bf16_bits(grid))
    s = Fraction(float(sc[0, 0]))
    assert np.all(sc == sc[0, 0])
    for r in range(rows.shape[0]):
        for j in range(64):
            v = Fraction(float(grid[r, j]))
            want = max(-8, min(7, _rne_int(_rn_f32(v / s))))
            assert codes[r, j] == want, (float(grid[r, j]), int(codes[r, j]), want)


def test_int4_dequant_error_bound():
    g = np.random.default_rng(5)
    x = O.f32_to_bf16_bits((g.standard_normal((33, 640)) * 3).astype(np.float32))
    codes, sc = O.quantize_int4_codes(x)
    xf = O.bf16_bits_to_f32(x).reshape(33, 10, 64).astype(np.float64)
    deq = codes.reshape(33, 10, 64).astype(np.float64) * sc.astype(np.float64)[..., None]
    assert np.all(np.abs(xf - deq) <= sc.astype(np.float64)[..., None] * (0.5 + 1e-6))
    assert codes.min() >= -7 and codes.max() <= 7  # symmetric scale amax/7 never reaches -8


def test_pack_layout_known_answer():
    codes = np.array([[1, -1, 7, -8, 0, 3]], np.int8)
    p = O.pack_int4(codes)
    assert p.tolist() == [[0xF1, 0x87, 0x30]]
    assert np.array_equal(O.unpack_int4(p), codes)
    g = np.random.default_rng(1)
    c = g.integers(-8, 8, size=(7, 256)).astype(np.int8)
    assert np.array_equal(O.unpack_int4(O.pack_int4(c)), c)


def test_group_psums_match_naive_loops():
    g = np.random.default_rng(2)
    qa = g.integers(0, 256, size=(5, 64), dtype=np.uint8)   # K = 128 -> 2 groups
    qw = g.integers(0, 256, size=(3, 64), dtype=np.uint8)
    ps = O.group_psums(qa, qw)
    assert ps.shape == (5, 3, 2)

    def nib(b, hi):
        v = (b >> 4) & 0xF if hi else b & 0xF
        return v - 16 if v >= 8 else v

    for m in range(5):
        for n in range(3):
            for gi in range(2):
                acc = 0
                for k in range(64 * gi, 64 * gi + 64):
                    acc += nib(int(qa[m, k // 2]), k % 2) * nib(int(qw[n, k // 2]), k % 2)
                assert ps[m, n, gi] == acc


# ---------------------------------------------------------------------------
# reference structural tests ported to the int4 oracle
# ---------------------------------------------------------------------------

def test_fold_to_dense_matches_two_branch():
    """tests/test_svdq_native_pgw685.py:163-191: the folded dense weight reproduces the two-branch linear."""
    g = np.random.default_rng(3)
    n, k, r = 256, 512, 32
    qw, sw = O.quantize_weight_int4(g.standard_normal((n, k)).astype(np.float32))
    smooth = O.f32_to_bf16_bits((g.random(k) + 0.5).astype(np.float32))
    down = O.f32_to_bf16_bits((g.standard_normal((k, r)) * 0.02).astype(np.float32))
    up = O.f32_to_bf16_bits((g.standard_normal((n, r)) * 0.02).astype(np.float32))
    x = g.standard_normal((8, k))
    w = O.fold_to_dense(qw, sw, smooth, down, up)
    got = x @ w.T
    xs = x / O.bf16_bits_to_f32(smooth).astype(np.float64)
    want = (xs @ O.dequantize_int4(qw, sw).T
            + (x @ O.bf16_bits_to_f32(down).astype(np.float64)) @ O.bf16_bits_to_f32(up).astype(np.float64).T)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-5


@pytest.mark.parametrize("shape", [(3072, 128), (9216, 128), (256, 3072)])
def test_int8_roundtrip_bound(shape):
    """tests/test_svdq_lowrank_quant_te148.py:92-107: int8 quantize->dequantize rel error < 0.02."""
    g = torch.Generator().manual_seed(2)
    w = (torch.randn(*shape, generator=g) * shape[0] ** -0.5).to(torch.bfloat16)
    bits = w.view(torch.int16).numpy().view(np.uint16)
    q, sa = O.quantize_act_int8(bits)
    back = q.astype(np.float64) * sa.astype(np.float64)
    ref = O.bf16_bits_to_f32(bits).astype(np.float64)
    assert np.linalg.norm(back - ref) / np.linalg.norm(ref) < 0.02


def test_int8_known_answers():
    x = np.zeros((3, 8), np.float32)
    x[0, :3] = [127.0, -63.5, 0.5]   # scale 1 -> codes 127, -64 (tie to even), 0
    x[1, :2] = [2.54, 1.27]
    x2 = O.f32_to_bf16_bits(x)
    q, sa = O.quantize_act_int8(x2)
    assert sa[0, 0] == 1.0 and q[0, :3].tolist() == [127, -64, 0]
    assert sa[2, 0] == np.float32(1e-12) and not q[2].any()
    v = O.bf16_bits_to_f32(x2)[1]
    s = np.float32(np.float32(np.abs(v).max()) / np.float32(127))
    assert sa[1, 0] == s and q[1, 0] == 127


def test_int8_exact_rational():
    g = np.random.default_rng(9)
    x = O.f32_to_bf16_bits((g.standard_normal((4, 256)) * 2).astype(np.float32))
    q, sa = O.quantize_act_int8(x)
    xf = O.bf16_bits_to_f32(x)
    for r in range(4):
        amax = Fraction(float(np.abs(xf[r]).max()))
        s = _rn_f32(amax / 127)
        assert Fraction(float(sa[r, 0])) == s
        for j in range(256):
            want = max(-127, min(127, _rne_int(_rn_f32(Fraction(float(xf[r, j])) / s))))
            assert q[r, j] == want


def test_int8_pertensor_and_static_known_answers():
    """The W8A8 quantizer's other modes (models/w8a8.py:261-273) on hand-computed rows: per-tensor takes
    the largest |x| of any row (rows with small values then quantize coarsely), a static scale is used as
    given (no clamp), and a static scale of 2^-3 turns multiples of 1/8 into their integer codes."""
    x = np.zeros((3, 8), np.float32)
    x[0, :3] = [127.0, -63.5, 0.5]
    x[1, :3] = [1.5, -2.5, 0.25]
    xb = O.f32_to_bf16_bits(x)
    q, sa = O.quantize_act_int8(xb, pertensor=True)
    assert sa.shape == (1, 1) and sa[0, 0] == 1.0
    assert q[0, :3].tolist() == [127, -64, 0] and q[1, :3].tolist() == [2, -2, 0] and not q[2].any()
    q, sa = O.quantize_act_int8(O.f32_to_bf16_bits(np.zeros((2, 8), np.float32)), pertensor=True)
    assert sa[0, 0] == np.float32(1e-12) and not q.any()
    codes = np.arange(-127, 129, dtype=np.int64).reshape(2, 128)
    codes[1, -1] = 500                                          # beyond the int8 range: clamps to 127
    xs = O.f32_to_bf16_bits((codes / 8.0).astype(np.float32))
    for pt in (False, True):
        q, sa = O.quantize_act_int8(xs, pertensor=pt, static=0.125)
        assert sa.shape == ((1, 1) if pt else (2, 1)) and (sa == np.float32(0.125)).all()
        assert q.astype(np.int64).tolist() == np.clip(codes, -127, 127).tolist()
    q, sa = O.quantize_act_int8(O.f32_to_bf16_bits(np.full((1, 8), 3.0, np.float32)), static=1e-20)
    assert sa[0, 0] == np.float32(1e-20) and (q == 127).all()   # no 1e-12 floor on a static scale


def test_int8_pertensor_exact_rational():
    """Per-tensor codes against exact rational arithmetic, with the tensor's scale from its largest |x|."""
    g = np.random.default_rng(19)
    xf = (g.standard_normal((5, 64)) * np.array([0.01, 1, 30, 0.5, 2])[:, None]).astype(np.float32)
    x = O.f32_to_bf16_bits(xf)
    q, sa = O.quantize_act_int8(x, pertensor=True)
    xv = O.bf16_bits_to_f32(x)
    s = _rn_f32(Fraction(float(np.abs(xv).max())) / 127)
    assert Fraction(float(sa[0, 0])) == s
    for r in range(5):
        for j in range(64):
            assert q[r, j] == max(-127, min(127, _rne_int(_rn_f32(Fraction(float(xv[r, j])) / s))))
    # the per-tensor scale is the largest per-token scale, and the row holding the maximum quantizes alike
    qr, sr = O.quantize_act_int8(x)
    assert sa[0, 0] == sr.max()
    top = int(np.argmax(sr[:, 0]))
    assert np.array_equal(q[top], qr[top])


def test_w8a8_linear_modes_agree_on_shared_scales():
    """With one row the per-tensor and per-token modes coincide, and a static scale equal to the dynamic
    one reproduces the dynamic output; the pertensor linear equals int GEMM x scalar x per-channel scale."""
    g = np.random.default_rng(23)
    x = O.f32_to_bf16_bits(g.standard_normal((1, 128)).astype(np.float32))
    qw, sw = O.quantize_weight_int8((g.standard_normal((32, 128)) * 0.05).astype(np.float32))
    y_tok = O.w8a8_linear(x, qw, sw, None)
    assert np.array_equal(O.w8a8_linear(x, qw, sw, None, pertensor=True), y_tok)
    _, sa = O.quantize_act_int8(x)
    assert np.array_equal(O.w8a8_linear(x, qw, sw, None, static=float(sa[0, 0])), y_tok)
    xm = O.f32_to_bf16_bits(g.standard_normal((6, 128)).astype(np.float32))
    qa, s = O.quantize_act_int8(xm, pertensor=True)
    want = (qa.astype(np.int64) @ qw.astype(np.int64).T) * float(s[0, 0]) * sw.astype(np.float64).reshape(1, -1)
    assert np.array_equal(O.w8a8_linear(xm, qw, sw, None, pertensor=True), want)


def test_w4a4_linear_reference_consistency():
    """The oracle's linear equals an independent float64 assembly of its documented formula."""
    g = np.random.default_rng(4)
    m, n, k, r = 16, 32, 128, 16
    x = O.f32_to_bf16_bits(g.standard_normal((m, k)).astype(np.float32))
    sm = O.f32_to_bf16_bits((g.random(k) + 0.5).astype(np.float32))
    qw, sw = O.quantize_weight_int4((g.standard_normal((n, k)) * 0.02).astype(np.float32))
    down = O.f32_to_bf16_bits((g.standard_normal((k, r)) * 0.02).astype(np.float32))
    up = O.f32_to_bf16_bits((g.standard_normal((n, r)) * 0.02).astype(np.float32))
    b = O.f32_to_bf16_bits((g.standard_normal(n) * 0.02).astype(np.float32))
    y = O.w4a4_linear(x, sm, qw, sw, down, up, b)
    qa, sa = O.quantize_act_int4(x, sm)
    ps = O.group_psums(qa, qw).astype(np.float64)             # [m, n, G]
    main = np.einsum("mng,mg,ng->mn", ps, sa.astype(np.float64), sw.astype(np.float64))
    la = O.round_bf16((O.bf16_bits_to_f32(x).astype(np.float64) @ O.bf16_bits_to_f32(down).astype(np.float64))
                      .astype(np.float32)).astype(np.float64)
    want = main + la @ O.bf16_bits_to_f32(up).astype(np.float64).T + O.bf16_bits_to_f32(b).astype(np.float64)
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# the package's offline producers agree with the oracle
# ---------------------------------------------------------------------------

def test_producers_match_oracle():
    from gen_worker_amd import svdq, w8a8

    g = torch.Generator().manual_seed(7)
    w = torch.randn(96, 320, generator=g) * 0.02
    w[3] = 0.0
    qw, sw = svdq.quantize_weight_int4(w)
    oq, osw = O.quantize_weight_int4(w.numpy())
    assert np.array_equal(qw.numpy(), oq) and np.array_equal(sw.numpy().view(np.uint16), osw.view(np.uint16))
    q8, s8 = w8a8.quantize_weight_int8(w)
    oq8, os8 = O.quantize_weight_int8(w.numpy())
    assert np.array_equal(q8.numpy(), oq8) and np.array_equal(s8.numpy(), os8)
    assert np.array_equal(svdq.unpack_int4(qw).numpy(), O.unpack_int4(oq))


# ---------------------------------------------------------------------------
# the float pieces: library routines and losslessly quantizable inputs
# ---------------------------------------------------------------------------

def _nibbles(packed: np.ndarray) -> np.ndarray:
    """Independent unpack: element 2j = low nibble of byte j, two's complement."""
    p = np.asarray(packed, np.int64)
    lo, hi = p & 0xF, p >> 4
    out = np.empty(p.shape[:-1] + (2 * p.shape[-1],), np.int64)
    out[..., 0::2], out[..., 1::2] = lo, hi
    return np.where(out >= 8, out - 16, out)


def test_gelu_tanh_matches_torch():
    y = np.linspace(-12.0, 12.0, 4001)
    want = torch.nn.functional.gelu(torch.from_numpy(y), approximate="tanh").numpy()
    assert np.allclose(O.gelu_tanh(y), want, rtol=1e-13, atol=1e-15)


def test_lowrank_down_matches_torch():
    g = np.random.default_rng(21)
    x = O.f32_to_bf16_bits(g.standard_normal((33, 320)).astype(np.float32))
    d = O.f32_to_bf16_bits((g.standard_normal((320, 16)) * 0.02).astype(np.float32))
    xt = torch.from_numpy(x.astype(np.int16)).view(torch.bfloat16).double()
    dt = torch.from_numpy(d.astype(np.int16)).view(torch.bfloat16).double()
    assert np.allclose(O.lowrank_down(x, d), (xt @ dt).numpy(), rtol=1e-12, atol=1e-14)


def test_int8_gemm_matches_torch():
    g = np.random.default_rng(22)
    qa = g.integers(-127, 128, size=(19, 257), dtype=np.int8)
    qw = g.integers(-127, 128, size=(23, 257), dtype=np.int8)
    want = (torch.from_numpy(qa).long() @ torch.from_numpy(qw).long().t()).numpy()
    assert np.array_equal(O.int8_gemm(qa, qw).astype(np.int64), want)
    assert int(O.int8_gemm(np.full((1, 64), -127, np.int8), np.full((1, 64), 127, np.int8))[0, 0]) == -64 * 127 * 127


def test_w8a8_linear_lossless_inputs():
    """Rows built as q * 2^-e with max |q| = 127 quantize losslessly (scale = 2^-e exactly), so the
    W8A8 linear must equal a plain float64 matmul of the inputs with the dequantized weights."""
    g = np.random.default_rng(23)
    m, n, k = 12, 40, 192
    q = g.integers(-127, 128, size=(m, k))
    q[:, 5] = 127
    e = g.integers(-3, 9, size=(m, 1))
    x = (q * np.exp2(-e.astype(np.float64))).astype(np.float32)
    xb = O.f32_to_bf16_bits(x)
    assert np.array_equal(O.bf16_bits_to_f32(xb), x)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    qw, sw = O.quantize_weight_int8(w)
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    want = x.astype(np.float64) @ (qw.astype(np.float64) * sw.astype(np.float64)).T + bias.astype(np.float64)
    assert np.allclose(O.w8a8_linear(xb, qw, sw, bias), want, rtol=1e-12, atol=1e-12)


def test_w8a8_pertensor_reference_roundings_match_torch():
    """The oracle's ``ref_roundings`` variant of the per-tensor branch equals the reference's statements run in
    torch (``models/w8a8.py:366-372``: ``_scaled_mm`` with unit ``scale_b`` to bf16, ``y * weight_scale.t()
    .to(y.dtype)``, ``y + bias`` in bf16), bit for bit; the per-token branch is unaffected by the flag."""
    g = np.random.default_rng(31)
    m, n, k = 24, 80, 192
    x = (g.standard_normal((m, k)) * 3).astype(np.float32)
    xb = O.f32_to_bf16_bits(x)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    qw, sw = O.quantize_weight_int8(w)
    bias = O.round_bf16((g.standard_normal(n) * 0.1).astype(np.float32))
    got = O.w8a8_linear(xb, qw, sw, bias, pertensor=True, ref_roundings=True)
    qa, sa = O.quantize_act_int8(xb, pertensor=True)
    acc = torch.from_numpy(qa).long() @ torch.from_numpy(qw).long().t()
    y = (acc.double() * float(sa[0, 0])).float().to(torch.bfloat16)          # _scaled_mm, scale_b = 1
    y = y * torch.from_numpy(sw).t().to(y.dtype)                              # weight scale in the output dtype
    y = y + torch.from_numpy(bias).to(torch.bfloat16)                         # bf16 bias
    assert np.array_equal(got, y.double().numpy())
    assert np.array_equal(O.w8a8_linear(xb, qw, sw, bias, ref_roundings=True), O.w8a8_linear(xb, qw, sw, bias))


def test_w8a8_pertensor_fused_epilogue_deviation_is_in_tolerance():
    """The int8 GEMM's per-tensor branch applies the weight scale and bias in fp32 in one epilogue and rounds
    once to bf16; the reference rounds three times in bf16. At config 0's shape (M=256, K=N=3072, 1% outlier
    channels x20), against the exact float64 product: the single rounding passes the north star's bar (the
    helpers' form: max-abs 2e-2 beyond the output's half-ulp rounding, mean-rel 5e-3, rel-Frobenius 2e-2);
    the reference's three roundings meet the mean-rel and rel-Frobenius bounds but not the max-abs one (its
    two extra roundings add up to another ulp on the largest outputs); the two are within mean-rel 5e-3 of
    each other."""
    from gen_worker_amd import synthetic
    from helpers import check_output

    c = synthetic.C0
    xb = synthetic.activation(c["m"], c["k"], outlier_frac=c["outlier_frac"], outlier_scale=c["outlier_scale"])
    xb = xb.view(torch.int16).numpy().view(np.uint16)
    L = synthetic.w8a8_layer(c["n"], c["k"])
    qw, sw = L.qweight.numpy(), L.weight_scale.numpy()
    bias = O.round_bf16(L.bias.float().numpy())
    exact = O.w8a8_linear(xb, qw, sw, bias, pertensor=True)
    fused = O.round_bf16(exact.astype(np.float32))
    ref = O.w8a8_linear(xb, qw, sw, bias, pertensor=True, ref_roundings=True).astype(np.float32)
    st_f = check_output(torch.from_numpy(fused).to(torch.bfloat16), exact, what="fused epilogue vs exact")
    r64 = ref.astype(np.float64)
    st_r = {"max_abs": O.max_abs_err(r64, exact), "mean_rel": O.mean_rel_err(r64, exact),
            "rel_fro": float(np.linalg.norm(r64 - exact) / np.linalg.norm(exact))}
    assert st_r["mean_rel"] <= 5e-3 and st_r["rel_fro"] <= 2e-2, st_r
    d = np.abs(fused.astype(np.float64) - ref)
    print(f"w8a8 pertensor vs exact: fused {st_f}; reference's three bf16 roundings {st_r}; between them: max "
          f"{d.max():.3e}, mean rel {O.mean_rel_err(fused, ref.astype(np.float64)):.3e}")
    assert st_f["mean_rel"] <= st_r["mean_rel"]
    assert O.mean_rel_err(fused, ref.astype(np.float64)) <= 5e-3


def test_w4a4_linear_lossless_inputs():
    """Groups built as q * 2^-e with max |q| = 7 quantize losslessly (fp16(amax/7) = 2^-e), and a
    power-of-two smoothing keeps that true, so the full linear (smoothing, quant, GEMM, second,
    low-rank, bias, GELU) must equal a plain float64 assembly from the inputs: x/smooth @ deq(W)^T.
    (s2 is pinned by the exact-rational scale and code tests.)"""
    g = np.random.default_rng(24)
    m, n, k, r = 10, 48, 256, 16
    grp = k // 64
    q = g.integers(-7, 8, size=(m, grp, 64))
    q[:, :, 3] = -7
    e = g.integers(-2, 6, size=(m, grp, 1))
    xs = (q * np.exp2(-e.astype(np.float64))).reshape(m, k)           # the smoothed activations
    sm = np.exp2(g.integers(-2, 3, size=k).astype(np.float64))         # power-of-two smoothing
    x = (xs * sm).astype(np.float32)
    xb, smb = O.f32_to_bf16_bits(x), O.f32_to_bf16_bits(sm.astype(np.float32))
    assert np.array_equal(O.bf16_bits_to_f32(xb).astype(np.float64), xs * sm)
    qw, sw = O.quantize_weight_int4((g.standard_normal((n, k)) * 0.02).astype(np.float32))
    wd = _nibbles(qw).astype(np.float64) * np.repeat(sw.astype(np.float64), 64, axis=1)
    down = O.f32_to_bf16_bits((g.standard_normal((k, r)) * 0.05).astype(np.float32))
    up = O.f32_to_bf16_bits((g.standard_normal((n, r)) * 0.05).astype(np.float32))
    b = O.f32_to_bf16_bits((g.standard_normal(n) * 0.1).astype(np.float32))
    second = (g.random(n) + 0.5).astype(np.float32)
    y = O.w4a4_linear(xb, smb, qw, sw, down, up, b, second=second, gelu=True)
    la = torch.from_numpy((x.astype(np.float64) @ O.bf16_bits_to_f32(down).astype(np.float64)).astype(np.float32))
    la = la.to(torch.bfloat16).double().numpy()
    pre = (xs @ wd.T) * second.astype(np.float64) + la @ O.bf16_bits_to_f32(up).astype(np.float64).T \
        + O.bf16_bits_to_f32(b).astype(np.float64)
    want = torch.nn.functional.gelu(torch.from_numpy(pre), approximate="tanh").numpy()
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)
