"""AWQ W4A16 modulation lane, CPU side: the oracle pinned by known answers, the product's format
functions against the oracle, and the host-side refusals of the packed module and op.

The reference holds no numeric AWQ fixtures; its own checks are structural (the packed module against the
decoded bf16 Linear, ``models/svdq_awq_packed.py:256-285``). The interleave is pinned here by where a
single code lands, the dequantized bf16 values by exact rational arithmetic, and the adaLN transform by
hand-computed rows and bias offsets.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits16
from oracle import awq_oracle as A
from oracle import svdq_oracle as O

from gen_worker_amd import awq


# ------------------------------------------------------------------ oracle pinning

@pytest.mark.parametrize("r,k", [(0, 0), (1, 0), (3, 5), (2, 9), (0, 31), (5, 32), (6, 63), (7, 64), (4, 100),
                                 (7, 127)])
def test_oracle_pack_one_hot_placement(r, k):
    """A single code (value 0xA) at (r, k) must land in the int16 word of packed row r // 4 at column
    64 (k // 64) + 16 (r % 4) + 8 ((k % 64) // 32) + k % 8, in nibble (k % 32) // 8: the word holds codes
    k, k + 8, k + 16, k + 24 of its 32-block, and the 16 words of a row's 64-column unit sit after the
    units of the lower rows of its group of four."""
    oc, ic = 8, 128
    codes = np.zeros((oc, ic), np.uint8)
    codes[r, k] = 0xA
    words = A.tinychat_pack(codes).view(np.uint16).reshape(oc // 4, ic)
    col = 64 * (k // 64) + 16 * (r % 4) + 8 * ((k % 64) // 32) + k % 8
    expect = np.zeros_like(words)
    expect[r // 4, col] = 0xA << (4 * ((k % 32) // 8))
    assert np.array_equal(words, expect)


def test_oracle_pack_roundtrip():
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (12, 192), dtype=np.uint8)
    assert np.array_equal(A.tinychat_unpack(A.tinychat_pack(codes), 12, 192), codes)


def test_oracle_num_scale_rows():
    # groups padded to packs of 8, pack count rounded up to 2 (g64) / 4 (g32)
    assert A.num_scale_rows(3072, 64) == 48       # 48 groups = 6 packs (already even)
    assert A.num_scale_rows(256, 64) == 16        # 4 groups -> 1 pack -> 2 packs
    assert A.num_scale_rows(64, 64) == 16
    assert A.num_scale_rows(3072, 32) == 96       # 96 groups = 12 packs (multiple of 4)
    assert A.num_scale_rows(15360, 64) == 240
    assert A.num_scale_rows(1088, 64) == 32       # 17 groups -> 3 packs -> 4
    assert A.num_scale_rows(256, 128) == 8        # other group sizes: packs of 8 only


def test_oracle_dequant_known_answers():
    bf = lambda v: int(O.f32_to_bf16_bits(np.array([v], np.float32))[0])
    # exact: 15 * 0.5 - 3.75 = 3.75; 0 * s + z = z
    assert A.dequant_exact_bf16_bits(15, bf(0.5), bf(-3.75)) == bf(3.75)
    assert A.dequant_exact_bf16_bits(0, bf(0.123), bf(-0.5)) == bf(-0.5)
    # rounding: 3 * 1.0078125 + 1 = 4.0234375 -> bf16 (8-bit significand, spacing 1/32 at 4) -> 4.03125
    assert A.dequant_exact_bf16_bits(3, bf(1.0078125), bf(1.0)) == bf(4.03125)
    # a bf16 tie after the fp32 sum: 1 * 1.0 + 2^-8 = 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> even (1.0)
    assert A.dequant_exact_bf16_bits(1, bf(1.0), bf(2.0 ** -8)) == bf(1.0)
    # ... and 3 * 2^-8 on top of 1 rounds up
    assert A.dequant_exact_bf16_bits(3, bf(2.0 ** -8), bf(1.0)) == bf(1.0 + 2.0 ** -6 * 1.0)


def test_oracle_dequant_matches_exact_arithmetic():
    """The vectorised fp32 path (product exact, one fp32 rounding of the sum, then bf16) against exact
    rational arithmetic over every code and a spread of scales / zeros of both signs."""
    rng = np.random.default_rng(1)
    s = O.f32_to_bf16_bits((rng.uniform(1e-3, 0.1, 24) * rng.choice([1, 1, 1, -1], 24)).astype(np.float32))
    z = O.f32_to_bf16_bits(rng.uniform(-0.8, 0.8, 24).astype(np.float32))
    codes = np.tile(np.arange(16, dtype=np.uint8), (24, 4))           # [24, 64]: every code, one group per row
    got = A.dequant_bf16_bits(codes, s.reshape(24, 1), z.reshape(24, 1))
    for r in range(24):
        for c in range(16):
            assert got[r, c] == A.dequant_exact_bf16_bits(c, int(s[r]), int(z[r])), (r, c)


def test_oracle_adanorm_known_answer():
    """6 splits over 12 rows: stored row j * 6 + s holds original row s * 2 + j; splits 1 and 4 gain +1."""
    w = np.arange(12, dtype=np.float64).reshape(12, 1)
    b = np.zeros(12)
    wo, bo = A.adanorm_apply(w, b, 6)
    assert wo[:, 0].tolist() == [0, 2, 4, 6, 8, 10, 1, 3, 5, 7, 9, 11]
    assert bo.tolist() == [0, 1, 0, 0, 1, 0] * 2
    w2, b2 = A.adanorm_undo(wo, bo, 6)
    assert np.array_equal(w2, w) and np.array_equal(b2, b)
    # two splits: 1 and splits - 2 = 0 both gain +1
    _, bo2 = A.adanorm_apply(np.zeros((4, 1)), np.zeros(4), 2)
    assert bo2.tolist() == [1, 1, 1, 1]


def test_oracle_linear_one_hot():
    """x = e_k picks column k of the bf16 weight, plus the bias."""
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, (16, 128), dtype=np.uint8)
    s = O.f32_to_bf16_bits(rng.uniform(1e-3, 0.05, (16, 2)).astype(np.float32))
    z = O.f32_to_bf16_bits(rng.uniform(-0.4, 0.0, (16, 2)).astype(np.float32))
    b = O.f32_to_bf16_bits(rng.normal(0, 0.1, 16).astype(np.float32))
    x = np.zeros((1, 128), np.uint16)
    x[0, 77] = O.f32_to_bf16_bits(np.array([1.0], np.float32))[0]
    y = A.awq_linear(x, codes, s, z, b)
    w = O.bf16_bits_to_f32(A.dequant_bf16_bits(codes, s, z))
    assert np.array_equal(y[0], w[:, 77].astype(np.float64) + O.bf16_bits_to_f32(b).astype(np.float64))


# ------------------------------------------------------------------ product format functions vs the oracle

@pytest.mark.parametrize("oc,ic", [(4, 64), (8, 128), (16, 320)])
def test_pack_matches_oracle(oc, ic):
    g = torch.Generator().manual_seed(oc * ic)
    codes = torch.randint(0, 16, (oc, ic), generator=g, dtype=torch.uint8)
    p = awq.pack_w4x16(codes)
    assert p.dtype == torch.int32 and tuple(p.shape) == (oc // 4, ic // 2)
    assert np.array_equal(p.numpy(), A.tinychat_pack(codes.numpy()))
    assert torch.equal(awq.unpack_w4x16(p, oc, ic), codes)


def test_num_scale_rows_matches_oracle():
    for ic, gs in ((3072, 64), (256, 64), (64, 64), (3072, 32), (15360, 64), (1088, 64), (256, 128)):
        assert awq.num_scale_rows(ic, gs) == A.num_scale_rows(ic, gs)


def test_adanorm_matches_oracle():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(36, 5, generator=g, dtype=torch.float64)
    b = torch.randn(36, generator=g, dtype=torch.float64)
    for splits in (2, 3, 6):
        wo, bo = awq.apply_adanorm_splits(w, b, splits)
        rw, rb = A.adanorm_apply(w.numpy(), b.numpy(), splits)
        assert np.array_equal(wo.numpy(), rw) and np.allclose(bo.numpy(), rb, rtol=0, atol=1e-12)
        wu, bu = awq.undo_adanorm_splits(wo, bo, splits)
        assert torch.equal(wu, w) and torch.allclose(bu.double(), b, rtol=0, atol=1e-6)


def test_encode_decode_roundtrip():
    """Exporter layout -> decoded bf16 Linear: the weight within half a quantization step (+ bf16 rounding)
    of the original, the bias back within bf16 rounding, the adaLN transform undone."""
    g = torch.Generator().manual_seed(4)
    w = torch.randn(96, 256, generator=g) * 0.05
    b = torch.randn(96, generator=g)
    for splits in (1, 6):
        t = awq.encode_awq_linear(w, b, adanorm_splits=splits)
        assert tuple(t["qweight"].shape) == (24, 128) and tuple(t["wscales"].shape) == (16, 96)
        assert awq.is_awq_linear(t)
        lin = awq.decode_awq_linear(t, 96, 256, adanorm_splits=splits)
        g4 = w.reshape(96, 4, 64)
        step = ((g4.amax(-1) - g4.amin(-1)) / 15.0).repeat_interleave(64, dim=1)
        lo = g4.amin(-1).abs().repeat_interleave(64, dim=1)
        err = (lin.weight.float() - w).abs()
        # half a step, plus the bf16 storage of scale (times a code <= 15) and zero, plus the bf16 weight
        bound = 0.5 * step + (15 * step + lo + w.abs()) * 2.0 ** -8 + 1e-6
        assert bool((err <= bound).all()), float((err - bound).max())
        # the stored bias is b (+1 on two splits) in bf16, the decoded one bf16 again: two roundings of |b| + 1
        assert bool(((lin.bias.float() - b).abs() <= (b.abs() + 1.0) * 2.0 ** -8).all())


def test_dequantize_matches_oracle():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(32, 128, generator=g) * 0.05
    t = awq.encode_awq_linear(w, None)
    deq = awq.dequantize_w4x16(t["qweight"], t["wscales"], t["wzeros"], 32, 128)
    codes = A.tinychat_unpack(t["qweight"].numpy(), 32, 128)
    s = bits16(t["wscales"][:2].t().contiguous())
    z = bits16(t["wzeros"][:2].t().contiguous())
    assert np.array_equal(deq.numpy(), A.dequant_f32(codes, s, z))


def test_scale_grid_refusals():
    g = torch.Generator().manual_seed(6)
    t = awq.encode_awq_linear(torch.randn(16, 256, generator=g), None)
    bad = t["wscales"].clone()
    bad[1] = 0                                        # a dead row before a live one
    with pytest.raises(awq.AwqLayoutError):
        awq.scales_and_zeros(bad, t["wzeros"], 16, 256)
    with pytest.raises(awq.AwqLayoutError):
        awq.unpack_w4x16(t["qweight"][:, :64], 16, 256)
    with pytest.raises(awq.AwqLayoutError):
        awq.decode_awq_linear({"qweight": t["qweight"]}, 16, 256)
    with pytest.raises(awq.AwqPackedError):
        awq.AwqPackedLinear(100, 24, bias=False)      # in % 128
    with pytest.raises(awq.AwqPackedError):
        awq.AwqPackedLinear(128, 24, bias=False)      # out % 16


def test_build_packed_module_layout():
    """The packed module's buffers: codes two per byte (even column low), grids [oc, groups], adaLN undone
    (checked against the decoded Linear's weight through the module's own bytes)."""
    g = torch.Generator().manual_seed(7)
    w = torch.randn(48, 256, generator=g) * 0.05
    b = torch.randn(48, generator=g)
    t = awq.encode_awq_linear(w, b, adanorm_splits=6)
    mod = awq.build_awq_packed_linear(t, 48, 256, adanorm_splits=6, device="cpu")
    lin = awq.decode_awq_linear(t, 48, 256, adanorm_splits=6)
    codes = torch.stack([mod.weight & 0xF, mod.weight >> 4], dim=-1).reshape(48, 256).float()
    deq = codes.reshape(48, 4, 64) * mod.wscales.float().unsqueeze(-1) + mod.wzeros.float().unsqueeze(-1)
    assert torch.equal(deq.reshape(48, 256).to(torch.bfloat16), lin.weight)
    assert torch.equal(mod.bias, lin.bias)


def test_op_refuses_cpu_and_bad_shapes():
    from gen_worker_amd.ops import SvdqOpError

    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    wt = torch.zeros(32, 128, dtype=torch.uint8)
    s = torch.zeros(32, 4, dtype=torch.bfloat16)
    with pytest.raises(SvdqOpError):
        torch.ops.cozy_gen_worker.awq_w4a16_mm(x, wt, s, s, None)        # CPU tensors


@pytest.mark.parametrize("splits", [1, 2, 3, 6])
def test_decoded_original_order_matches_dense_undo(splits):
    """The decoder's row reorder and bias fix (on codes and grids) equal the dense inverse transform applied
    to the dequantized stored weight, for every split count (3: the two shifted splits coincide)."""
    g = torch.Generator().manual_seed(40 + splits)
    oc, ic = 48, 128
    t = awq.encode_awq_linear(torch.randn(oc, ic, generator=g) * 0.05, torch.randn(oc, generator=g),
                              adanorm_splits=splits)
    stored = awq.decode_awq_tensors(t, oc, ic)
    assert stored.group_size == 64 and (stored.out_features, stored.in_features) == (oc, ic)
    dec = stored.in_original_order(splits)
    w_ref, b_ref = awq.undo_adanorm_splits(stored.weight(), t["bias"], splits)
    assert torch.equal(dec.weight(), w_ref)
    assert torch.equal(dec.bias, b_ref.float() if splits > 1 else t["bias"])
