"""GPU tests at the QKV projection shape (K=3072 -> N=9216) over the token counts of the M sweep
(256, 1024, 4608, 16384), for the W4A4 module (bf16 and fp16 outputs) and the W8A8 module.

Every linear here is token-local (each output row depends on its own input row only), so the oracle's
float64 linear (``oracle/svdq_oracle.py``) runs on a row sample: the first rows, the rows either side of
the 256- and 288-row tile edges, and the last rows. The full outputs are checked for properties that need
no oracle: finite, deterministic run to run, and (W4A4) within tolerance of the general int8-MFMA lane,
which computes the same linear with a different kernel and accumulation order.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits16, check_output
from oracle import svdq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
K, N, R = 3072, 9216, 32


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native

    _native.load()
    assert torch.cuda.is_available()
    yield


@pytest.fixture(scope="module")
def w4a4_layer():
    from gen_worker_amd import synthetic

    return synthetic.w4a4_layer(N, K, R)


@pytest.fixture(scope="module")
def w8a8_layer():
    from gen_worker_amd import synthetic

    return synthetic.w8a8_layer(N, K)


def _rows(m):
    r = np.r_[0:6, 255:258, 287:290, 1023:1026, 2303:2306, 4607:4610, m - 6:m]
    return np.unique(r[r < m])


def _act(m):
    from gen_worker_amd import synthetic

    return synthetic.activation(m, K, outlier_frac=0.005, outlier_scale=30.0, seed=1000 + m)


@pytest.mark.parametrize("m", [256, 1024, 4608, 16384])
@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_w4a4_qkv(m, odt, w4a4_layer):
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    L = w4a4_layer
    kw = dict(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down, proj_up=L.proj_up,
              bias=L.bias, out_dtype=odt, device=DEV)
    mod = build_svdq_w4a4_linear(**kw)
    assert mod.lane == "fp6"
    x = _act(m).to(DEV)
    y = mod(x)
    y2 = mod(x)
    torch.cuda.synchronize()
    assert y.dtype == odt and tuple(y.shape) == (m, N)
    assert torch.isfinite(y).all()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "not deterministic"
    rows = _rows(m)
    ref = O.w4a4_linear(bits16(x[rows]), bits16(L.smooth), L.qweight.numpy(), L.wscales.numpy(),
                        bits16(L.proj_down), bits16(L.proj_up), bits16(L.bias))
    check_output(y[rows], ref, what=f"W4A4 QKV M={m} {odt}")
    if m <= 4608:
        # the general int8-MFMA lane (int4 nibble operands, a different kernel) on the full output
        cg = torch.ops.cozy_gen_worker
        qa, sa, la = cg.svdq_quant_lora(x, mod.smooth_factor, None, mod.proj_down_op)
        yg = cg.svdq_w4a4_linear(qa, sa, mod.weight, mod.weight_scale, None, mod.second, la, mod.proj_up, mod.bias,
                                 odt, False)
        d = (y.float() - yg.float()).abs()
        scale = yg.float().abs().mean().item()
        assert d.mean().item() <= 5e-3 * scale, f"lanes disagree: mean {d.mean().item()} vs {scale}"


@pytest.mark.parametrize("m", [256, 1024, 4608, 16384])
@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("mode", ["rowwise", "pertensor"])
def test_w8a8_qkv(m, odt, mode, w8a8_layer):
    from gen_worker_amd.w8a8 import build_int8_linear

    L = w8a8_layer
    mod = build_int8_linear(qweight=L.qweight, weight_scale=L.weight_scale, bias=L.bias, compute_dtype=odt,
                            device=DEV, gemm_mode=mode)
    x = _act(m).to(DEV)
    y = mod(x)
    y2 = mod(x)
    torch.cuda.synchronize()
    assert y.dtype == odt and tuple(y.shape) == (m, N) and torch.isfinite(y).all()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "not deterministic"
    if mode == "pertensor":
        # one activation scale for the whole call: the oracle needs every row's absmax, then checks a sample
        xs = bits16(x)
        amax = float(np.abs(O.bf16_bits_to_f32(xs)).max())
        static = max(np.float32(amax) / np.float32(O.INT8_QMAX), np.float32(O.INT8_SCALE_MIN))
        rows = _rows(m)
        ref = O.w8a8_linear(xs[rows], L.qweight.numpy(), L.weight_scale.numpy(), L.bias.numpy(), pertensor=True,
                            static=float(static))
    else:
        rows = _rows(m)
        ref = O.w8a8_linear(bits16(x[rows]), L.qweight.numpy(), L.weight_scale.numpy(), L.bias.numpy())
    check_output(y[rows], ref, what=f"W8A8 QKV M={m} {odt} {mode}")


def test_w8a8_gate_on_the_device():
    """The W8A8 branch gate (``models/w8a8.py:137-256``) on MI355X: both branches' probes pass, their 4096^3
    timings under both protocols are recorded for every branch it tried, and the mode follows its rule (the
    first branch at >= 1.10x over bf16, else the dequant lane)."""
    from gen_worker_amd import qualify

    for mode in qualify.W8A8_MODES:
        assert qualify.w8a8_probe(mode) is None, mode
    q = qualify.qualify_w8a8()
    print("w8a8 qualification", q)
    tried = list(q.timings)
    assert tried and tried[0] == "rowwise"
    for mode, t in q.timings.items():
        assert set(t) == {"graph", "eager"} and all(v[0] > 0 and v[1] > 0 for v in t.values())
    first_ok = next((m_ for m_ in qualify.W8A8_MODES if m_ in q.timings
                     and q.timings[m_]["graph"][2] >= qualify.BENCH_MIN_SPEEDUP), "")
    assert q.mode == first_ok, q
