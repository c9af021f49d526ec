"""GPU tests of the W8A8 lane's three activation-scale modes (the reference's ``quantize(x2, pertensor,
static)``, ``models/w8a8.py:261-273``, and the two ``_scaled_mm`` branches, ``:366-378``): codes and scales
bit-exact against the oracle (``oracle/svdq_oracle.py`` ``quantize_act_int8``), outputs within the
north-star tolerance of the oracle's float64 linear, and the module's ``gemm_mode`` / ``input_scale``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits16, check_output, from_bits
from oracle import svdq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
MODES = [("rowwise", None), ("pertensor", None), ("rowwise", 0.05), ("pertensor", 0.03)]


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native

    _native.load()
    assert torch.cuda.is_available()
    yield


def _act(m, k, seed):
    g = np.random.default_rng(seed)
    x = (g.standard_normal((m, k)) * np.exp(g.uniform(-3, 2, (m, 1)))).astype(np.float32)
    x[:, g.integers(0, k, 4)] *= 25.0
    if m > 3:
        x[3] = 0.0                          # an all-zero row
    return O.f32_to_bf16_bits(x)


def _quant(xb, mode, static):
    st = torch.tensor([[static]], dtype=torch.float32, device=DEV) if static is not None else None
    return torch.ops.cozy_gen_worker.w8a8_quant(from_bits(xb, torch.bfloat16, DEV), mode == "pertensor", st)


@pytest.mark.parametrize("mode,static", MODES)
@pytest.mark.parametrize("m,k", [(1, 64), (37, 448), (300, 3072), (4608, 3072)])
def test_quant_modes_bit_exact(mode, static, m, k):
    xb = _act(m, k, seed=m + k)
    q, sa = _quant(xb, mode, static)
    wq, wsa = O.quantize_act_int8(xb, pertensor=mode == "pertensor", static=static)
    torch.cuda.synchronize()
    assert tuple(sa.shape) == wsa.shape
    assert np.array_equal(sa.cpu().numpy(), wsa), f"{mode} static={static}: scales differ"
    assert np.array_equal(q.cpu().numpy(), wq), f"{mode} static={static}: codes differ"


def test_pertensor_amax_cell_is_rezeroed():
    """The per-tensor maximum is folded atomically into a cell the call clears first: a large tensor, then a
    small one, must not carry the first maximum over."""
    big = _act(64, 256, seed=1)
    small = O.f32_to_bf16_bits(np.full((4, 256), 0.5, np.float32))
    _quant(big, "pertensor", None)
    q, sa = _quant(small, "pertensor", None)
    wq, wsa = O.quantize_act_int8(small, pertensor=True)
    assert np.array_equal(sa.cpu().numpy(), wsa) and np.array_equal(q.cpu().numpy(), wq)


@pytest.mark.parametrize("mode,static", MODES)
def test_scaled_mm_modes_match_oracle(mode, static):
    m, n, k = 300, 400, 1024
    g = np.random.default_rng(5)
    xb = _act(m, k, seed=11)
    qw, sw = O.quantize_weight_int8((g.standard_normal((n, k)) * 0.02).astype(np.float32))
    b = (g.standard_normal(n) * 0.02).astype(np.float32)
    q, sa = _quant(xb, mode, static)
    for bias, odt in ((torch.from_numpy(b).to(DEV), torch.bfloat16), (None, torch.float16)):
        y = torch.ops.cozy_gen_worker.w8a8_scaled_mm(q, torch.from_numpy(qw).to(DEV), sa,
                                                     torch.from_numpy(sw).to(DEV), bias, odt)
        ref = O.w8a8_linear(xb, qw, sw, b if bias is not None else None, pertensor=mode == "pertensor",
                            static=static)
        check_output(y, ref, what=f"w8a8 {mode} static={static}")


@pytest.mark.parametrize("mode,static", MODES)
def test_module_modes(mode, static):
    from gen_worker_amd import synthetic
    from gen_worker_amd.w8a8 import build_int8_linear

    L = synthetic.w8a8_layer(512, 1024)
    st = torch.tensor([[static]]) if static is not None else None
    mod = build_int8_linear(qweight=L.qweight, weight_scale=L.weight_scale, bias=L.bias, device=DEV,
                            input_scale=st, gemm_mode=mode)
    assert ("input_scale" in mod.state_dict()) == (static is not None)
    assert f"gemm_mode={mode}" in repr(mod)
    x = synthetic.activation(2 * 96, 1024, outlier_frac=0.01, outlier_scale=20.0)
    y = mod(x.to(DEV).reshape(2, 96, 1024))
    assert tuple(y.shape) == (2, 96, 512)
    ref = O.w8a8_linear(bits16(x), L.qweight.numpy(), L.weight_scale.numpy(), L.bias.numpy(),
                        pertensor=mode == "pertensor", static=static)
    check_output(y.reshape(-1, 512), ref, what=f"module {mode} static={static}")

