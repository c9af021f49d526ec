"""GPU parity of the AWQ W4A16 modulation lane: the dequantized bf16 weight bit for bit against the oracle,
the op's output against the float64 oracle product (tolerance of tests/helpers.py), the reference's own
packed-vs-decoded check, the adaLN path at the Flux modulation shape, and determinism."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits16, check_output, from_bits
from oracle import awq_oracle as A
from oracle import svdq_oracle as O

from gen_worker_amd import awq
from gen_worker_amd.ops import AWQ_GEMV_MAX_M, SvdqOpError

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(n: int, k: int, seed: int, bias: bool = True):
    """Random codes, positive scales and negative pre-scaled zeros in the ranges an exporter writes."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    s = O.f32_to_bf16_bits(rng.uniform(0.002, 0.01, (n, k // 64)).astype(np.float32))
    z = O.f32_to_bf16_bits(-rng.uniform(0.0, 0.08, (n, k // 64)).astype(np.float32))
    b = O.f32_to_bf16_bits(rng.normal(0, 0.5, n).astype(np.float32)) if bias else None
    packed = (codes[:, 1::2] << 4) | codes[:, 0::2]
    t = dict(weight=torch.from_numpy(packed).to(DEV), wscales=from_bits(s, torch.bfloat16, DEV),
             wzeros=from_bits(z, torch.bfloat16, DEV),
             bias=from_bits(b, torch.bfloat16, DEV) if bias else None)
    return codes, s, z, b, t


@pytest.mark.parametrize("n,k", [(16, 128), (512, 256), (768, 3072), (3072, 3072)])
def test_dequant_bit_exact(n, k):
    codes, s, z, _, t = _layer(n, k, seed=n + k, bias=False)
    w = torch.ops.cozy_gen_worker.awq_w4a16_dequant(t["weight"], t["wscales"], t["wzeros"])
    assert np.array_equal(bits16(w), A.dequant_bf16_bits(codes, s, z))


@pytest.mark.parametrize("m,n,k,bias", [(1, 16, 128, True), (1, 512, 256, False), (2, 768, 3072, True),
                                        (3, 3072, 3072, True), (4, 256, 1024, True), (5, 512, 3072, False),
                                        (16, 256, 512, True), (17, 256, 512, True), (1, 18432, 3072, True)])
def test_mm_matches_oracle(m, n, k, bias):
    codes, s, z, b, t = _layer(n, k, seed=7 * m + n + k, bias=bias)
    g = torch.Generator().manual_seed(m * 1000 + k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    y = torch.ops.cozy_gen_worker.awq_w4a16_mm(x.to(DEV), t["weight"], t["wscales"], t["wzeros"], t["bias"])
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, n)
    ref = A.awq_linear(bits16(x), codes, s, z, b)
    check_output(y, ref, what=f"awq m={m} n={n} k={k} ({'gemv' if m <= AWQ_GEMV_MAX_M else 'dequant + gemm'})")


def test_mm_deterministic_and_row_independent():
    """Repeated calls agree bit for bit, and a row's result does not depend on the other rows of its chunk."""
    _, _, _, _, t = _layer(1024, 3072, seed=3)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 3072, generator=g).to(torch.bfloat16).to(DEV)
    op = torch.ops.cozy_gen_worker.awq_w4a16_mm
    y1 = op(x, t["weight"], t["wscales"], t["wzeros"], t["bias"])
    y2 = op(x, t["weight"], t["wscales"], t["wzeros"], t["bias"])
    assert torch.equal(y1, y2)
    for r in range(4):
        yr = op(x[r:r + 1].contiguous(), t["weight"], t["wscales"], t["wzeros"], t["bias"])
        assert torch.equal(yr[0], y1[r])


def test_packed_self_check():
    """The reference's packed-lane gate (models/svdq_awq_packed.py:256-285)."""
    assert awq.awq_packed_self_check(DEV) is None


def test_flux_modulation_shape_with_adanorm():
    """A dual-block modulation layer (3072 -> 6 x 3072, six adaLN splits) from exporter-layout tensors: the
    packed module against the oracle on the module's own bytes and against the decoded bf16 Linear."""
    g = torch.Generator().manual_seed(11)
    w = torch.randn(18432, 3072, generator=g) * 0.02
    b = torch.randn(18432, generator=g) * 0.02
    tensors = awq.encode_awq_linear(w, b, adanorm_splits=6)
    mod = awq.build_awq_packed_linear(tensors, 18432, 3072, adanorm_splits=6, device=DEV)
    lin = awq.decode_awq_linear(tensors, 18432, 3072, adanorm_splits=6, device=DEV)
    x = torch.randn(1, 3072, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        y = mod(x.to(DEV))
        yl = lin(x.to(DEV))
    wb = mod.weight.cpu().numpy()
    codes = np.stack([wb & 0xF, wb >> 4], axis=-1).reshape(18432, 3072).astype(np.uint8)
    ref = A.awq_linear(bits16(x), codes, bits16(mod.wscales), bits16(mod.wzeros), bits16(mod.bias))
    check_output(y, ref, what="flux modulation 3072->18432")
    rel = ((y.float() - yl.float()).norm() / yl.float().norm()).item()
    assert rel <= 5e-3, rel


def test_mm_refusals():
    _, _, _, _, t = _layer(256, 256, seed=1)
    x = torch.zeros(1, 256, dtype=torch.bfloat16, device=DEV)
    op = torch.ops.cozy_gen_worker.awq_w4a16_mm
    with pytest.raises(SvdqOpError):
        op(torch.zeros(1, 384, dtype=torch.bfloat16, device=DEV), t["weight"], t["wscales"], t["wzeros"], None)
    with pytest.raises(SvdqOpError):
        op(x, t["weight"], t["wscales"][:, :2].contiguous(), t["wzeros"], None)
    with pytest.raises(SvdqOpError):
        op(x.float(), t["weight"], t["wscales"], t["wzeros"], None)
    assert op(x[:0], t["weight"], t["wscales"], t["wzeros"], None).shape == (0, 256)
