"""GPU coverage of every output tile of the fp6 GEMM (``gwa_svdq_gemm_w4a4_fp6``).

The tile model picks one shape per (M, N); ``gwa_svdq_gemm_w4a4_fp6_force_tile`` pins one so that each tile
(the fp6 kernel's 256 x 256, 256 x 128, 128 x 128, 192 x 256 and the pipelined 288 x 192, 256 x 192) runs
on ragged shapes, every rank, both output dtypes, GELU and a per-channel second scale. All tiles issue the
same fp32 operations per output element in the same order, so their outputs must agree bit for bit; each is
also checked against the oracle's dequantize-then-matmul (``oracle/svdq_oracle.py``) on a row sample.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits16, check_output
from oracle import svdq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TILES = {0: (256, 256), 1: (256, 128), 2: (128, 128), 3: (192, 256), 4: (288, 192), 5: (256, 192), 6: (64, 128)}


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
    yield lib.gwa_svdq_gemm_w4a4_fp6_force_tile
    lib.gwa_svdq_gemm_w4a4_fp6_force_tile(-1)


def _layer_case(m, n, k, r, seed, per_channel=False):
    from gen_worker_amd import synthetic
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    L = synthetic.w4a4_layer(n, k, r, seed_offset=seed)
    mod = build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                 proj_up=L.proj_up, bias=L.bias, device=DEV)
    x = synthetic.activation(m, k, outlier_frac=0.005, outlier_scale=30.0, seed=seed).to(DEV)
    second = None
    if per_channel:
        second = np.linspace(0.5, 2.0, n).astype(np.float32)
    cg = torch.ops.cozy_gen_worker
    q6, la = cg.svdq_quant_fp6(x, mod.smooth_factor, None, mod.proj_down_op6 if r else None)
    sec = torch.from_numpy(second).to(DEV) if second is not None else mod.second

    def gemm(out_dtype, gelu):
        return cg.svdq_w4a4_linear_fp6(q6, mod.weight_fp6, None, sec, la if r else None,
                                       mod.proj_up if r else None, mod.bias, out_dtype, gelu)

    def oracle(rows, gelu):
        return O.w4a4_linear(bits16(x[rows]), bits16(L.smooth), L.qweight.numpy(), L.wscales.numpy(),
                             bits16(L.proj_down) if r else None, bits16(L.proj_up) if r else None, bits16(L.bias),
                             second=second, gelu=gelu)

    return gemm, oracle


def _sample_rows(m, tm):
    """First and last rows, and the rows either side of every tile boundary (capped)."""
    rows = set(range(min(m, 24))) | set(range(max(0, m - 24), m))
    for b in range(tm, m, tm)[:6]:
        rows |= {b - 1, b}
    return np.array(sorted(rows))


# (m, n, k, rank, gelu, out dtype, per-channel second): ragged in both dimensions for every tile shape
_CASES = [
    (577, 656, 384, 32, False, torch.bfloat16, False),
    (1, 48, 128, 0, False, torch.bfloat16, False),
    (300, 400, 256, 64, True, torch.float16, False),
    (290, 208, 128, 128, False, torch.bfloat16, True),
    (613, 1040, 640, 16, True, torch.bfloat16, True),
    (333, 464, 448, 32, False, torch.bfloat16, False),   # K % 128 == 64: the records end in a half stage
]


@pytest.mark.parametrize("case", _CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}r{c[3]}")
def test_every_tile_agrees_and_matches_oracle(case, force):
    m, n, k, r, gelu, odt, pc = case
    gemm, oracle = _layer_case(m, n, k, r, seed=m + n + r, per_channel=pc)
    outs = {}
    for t, (tm, _tn) in TILES.items():
        force(t)
        outs[t] = gemm(odt, gelu)
    force(-1)
    torch.cuda.synchronize()
    first = outs[0]
    assert first.dtype == odt and tuple(first.shape) == (m, n)
    for t, y in outs.items():
        assert torch.equal(y.view(torch.int16), first.view(torch.int16)), f"tile {TILES[t]} differs from 256x256"
    rows = _sample_rows(m, 96)
    check_output(first[rows], oracle(rows, gelu), what=f"fp6 tiles {m}x{n}x{k} r{r}")


@pytest.mark.parametrize("m,n", [(4608, 3072), (4096, 3072), (1024, 3072), (4608, 9216)])
def test_model_tiles_at_layer_shapes(m, n, force):
    """The DiT layer shapes at K=3072, rank 32: the model's tile and the pipelined tiles equal the 256 x 256
    tile bit for bit, and the output matches the oracle on rows around the 288- and 256-row tile edges."""
    from gen_worker_amd import _native

    lib = _native.load()
    picked = lib.gwa_svdq_gemm_w4a4_fp6_tile(m, n)
    assert picked in TILES
    gemm, oracle = _layer_case(m, n, 3072, 32, seed=7)
    force(0)
    base = gemm(torch.bfloat16, False)
    outs = {}
    for t in sorted({picked, 4, 5}):
        force(t)
        outs[t] = gemm(torch.bfloat16, False)
    force(-1)
    torch.cuda.synchronize()
    for t, y in outs.items():
        assert torch.equal(y.view(torch.int16), base.view(torch.int16)), f"{m}x{n}: tile {TILES[t]} differs"
    rows = np.unique(np.r_[0:8, 255:258, 287:290, 2303:2306, m - 8:m])
    rows = rows[rows < m]
    check_output(base[rows], oracle(rows, False), what=f"fp6 {m}x{n}x3072")
