"""GPU coverage of every output tile of the W8A8 GEMM (``gwa_w8a8_gemm``).

The GEMM picks 256 x 256 tiles (direct-to-LDS copies, eight waves; stages of 64 or 128 K-bytes) when they
give every CU a tile, else 128 x 128 (register-staged copies); ``gwa_w8a8_gemm_force_tile`` pins one. All
accumulate the exact int32 dot product and apply the same fp32 epilogue, so their outputs must agree bit for
bit on ragged shapes,
short K (one to three stages, fewer than the copy pipeline's depth), both scale modes, every bias dtype and
both output dtypes; each is also checked against the oracle's float64 linear (``oracle/svdq_oracle.py``
``w8a8_linear``, the reference's ``_scaled_mm`` epilogue of ``models/w8a8.py:366-378``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import check_output
from oracle import svdq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMALL, LARGE = 0, 1  # GWA_W8A8_TILE_128x128, GWA_W8A8_TILE_256x256


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native

    _native.load()
    assert torch.cuda.is_available()
    yield


@pytest.fixture
def force():
    from gen_worker_amd import _native

    lib = _native.load()
    yield lib.gwa_w8a8_gemm_force_tile
    lib.gwa_w8a8_gemm_force_tile(-1)


def _operands(m, n, k, seed, pertensor):
    g = np.random.default_rng(seed)
    x = (g.standard_normal((m, k)) * np.exp(g.uniform(-2, 1, (m, 1)))).astype(np.float32)
    x[:, g.integers(0, k, 3)] *= 20.0
    xb = O.f32_to_bf16_bits(x)
    qa, sa = O.quantize_act_int8(xb, pertensor=pertensor)
    qw, sw = O.quantize_weight_int8((g.standard_normal((n, k)) * 0.02).astype(np.float32))
    b = (g.standard_normal(n) * 0.05).astype(np.float32)
    return xb, qa, sa, qw, sw, b


def _bias(b, dt):
    if dt is None:
        return None
    return torch.from_numpy(b).to(DEV).to(dt)


def _run(qa, sa, qw, sw, bias, odt):
    return torch.ops.cozy_gen_worker.w8a8_scaled_mm(torch.from_numpy(qa).to(DEV), torch.from_numpy(qw).to(DEV),
                                                    torch.from_numpy(np.ascontiguousarray(sa)).to(DEV),
                                                    torch.from_numpy(sw).to(DEV), bias, odt)


# (m, n, k, pertensor, bias dtype, out dtype): ragged m / n around 256, K of 1, 2, 3 and many stages, and
# K = 192 (not a whole stage)
_CASES = [
    (1, 16, 128, False, torch.float32, torch.bfloat16),
    (64, 512, 256, False, None, torch.bfloat16),
    (130, 784, 128, True, torch.bfloat16, torch.float16),
    (257, 272, 384, False, torch.float16, torch.bfloat16),
    (300, 400, 1024, False, torch.float32, torch.float16),
    (513, 1040, 3072, True, torch.bfloat16, torch.bfloat16),
    (257, 272, 192, False, torch.float16, torch.bfloat16),
]


@pytest.mark.parametrize("m,n,k,pertensor,bdt,odt", _CASES)
def test_tiles_agree_and_match_oracle(force, m, n, k, pertensor, bdt, odt):
    xb, qa, sa, qw, sw, b = _operands(m, n, k, seed=m + n + k, pertensor=pertensor)
    bias = _bias(b, bdt)
    outs = {}
    for tile in (SMALL, LARGE):
        force(tile)
        outs[tile] = _run(qa, sa, qw, sw, bias, odt)
    torch.cuda.synchronize()
    assert torch.equal(outs[SMALL], outs[LARGE]), f"tiles differ at {(m, n, k)}"
    bref = None if bdt is None else bias.float().cpu().numpy()
    ref = O.w8a8_linear(xb, qw, sw, bref, pertensor=pertensor)
    check_output(outs[LARGE], ref, what=f"w8a8 256x256 tile {(m, n, k)}")


def test_large_shapes_take_the_large_tile_and_agree(force):
    """QKV at 4608 tokens (648 tiles of 256 x 256): the default choice is the large tile; it agrees bit for bit
    with the forced 128 x 128 tile and with an exact float64 product of the codes on the GPU."""
    from gen_worker_amd import _native

    m, n, k = 4608, 9216, 3072
    assert _native.load().gwa_w8a8_gemm_tile(m, n, k) == LARGE
    g = torch.Generator(device=DEV).manual_seed(7)
    qa = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=DEV, generator=g)
    qw = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=DEV, generator=g)
    sa = torch.rand(m, device=DEV, generator=g) * 1e-3 + 1e-4
    sw = torch.rand(n, device=DEV, generator=g) * 1e-3 + 1e-4
    bias = torch.randn(n, device=DEV, generator=g)
    cg = torch.ops.cozy_gen_worker
    y = cg.w8a8_scaled_mm(qa, qw, sa, sw, bias, torch.bfloat16)
    for tile in (SMALL, LARGE):
        force(tile)
        assert torch.equal(y, cg.w8a8_scaled_mm(qa, qw, sa, sw, bias, torch.bfloat16)), f"tile {tile}"
    # |dot| <= 127^2 * 3072 < 2^53: the float64 product is exact; rows sampled across tile boundaries
    rows = torch.tensor([0, 1, 255, 256, 2047, 2048, 4351, 4352, 4607], device=DEV)
    acc = qa[rows].double() @ qw.double().t()
    ref = (acc.float() * sa[rows, None] * sw[None, :] + bias[None, :]).double().cpu().numpy()
    check_output(y[rows], ref, what="w8a8 QKV 4608")
