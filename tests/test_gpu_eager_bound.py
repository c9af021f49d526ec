"""The modules' eager forwards through their bound calls (ops.BoundLinearFp6, ops.BoundLinearW8a8) against the ops.

``SvdqW4A4Linear.forward`` in eager mode calls the library entry points of ``svdq_forward_fp6`` /
``svdq_forward_gemv`` directly with the operands bound once. These tests hold it to the ops bit for bit over
the token counts on both sides of the GEMV bound, the epilogue variants and the output dtypes; check that a
changed operand, output dtype or activation rebinds; and that a dispatch mode routes the forward through the
op with the same result.
"""

from __future__ import annotations

import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode

pytestmark = pytest.mark.gpu
DEV = "cuda"
K, N = 640, 384   # K % 128 == 0 (the fp6 lane), N % 16 == 0


@pytest.fixture(scope="module", autouse=True)
def _lib():
    from gen_worker_amd import _native

    _native.load()
    assert torch.cuda.is_available()
    yield


def _module(rank, bias, activation=None, out_dtype=None, per_channel=False, seed=3):
    from gen_worker_amd import synthetic
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    L = synthetic.w4a4_layer(N, K, rank or 16, seed_offset=seed)
    second = None
    if per_channel:
        g = torch.Generator().manual_seed(seed)
        second = torch.rand(N, generator=g) + 0.5
    return build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth,
                                  proj_down=L.proj_down if rank else None, proj_up=L.proj_up if rank else None,
                                  bias=L.bias if bias else None, second=second, activation=activation,
                                  out_dtype=out_dtype, device=DEV)


def _op(mod, x):
    """The module's forward as the registered ops compute it."""
    cg = torch.ops.cozy_gen_worker
    odt = mod.out_dtype or torch.bfloat16
    gelu = mod.activation == "gelu_tanh"
    pdo6 = mod.proj_down_op6 if mod.rank else None
    up = mod.proj_up if mod.rank else None
    if x.shape[0] <= mod._gemv_max_m and x.shape[0] > 0:
        return cg.svdq_forward_gemv(x, mod.smooth_factor, None, pdo6, mod.weight, mod.weight_scale, mod.second, up,
                                    mod.bias, odt, gelu)
    return cg.svdq_forward_fp6(x, mod.smooth_factor, None, pdo6, mod.weight_fp6, mod.second, up, mod.bias, odt,
                               gelu)


def _act(m, seed=7):
    from gen_worker_amd import synthetic

    return synthetic.activation(m, K, outlier_frac=0.005, outlier_scale=30.0, seed=seed + m).to(DEV)


@pytest.mark.parametrize("rank,bias,activation,out_dtype,per_channel", [
    (32, True, None, None, False),
    (0, False, None, None, False),
    (16, True, "gelu_tanh", torch.float16, True),
    (64, False, None, torch.float16, False),
])
def test_bound_forward_equals_the_ops(rank, bias, activation, out_dtype, per_channel):
    mod = _module(rank, bias, activation, out_dtype, per_channel)
    assert mod.lane == "fp6" and mod._gemv_max_m > 0
    ms = sorted({0, 1, 3, mod._gemv_max_m, mod._gemv_max_m + 1, 77, 300})
    for m in ms:
        x = _act(m)
        y = mod(x)
        assert mod._bound is not None, "the eager forward did not take the bound call"
        ref = _op(mod, x)
        torch.cuda.synchronize()
        assert y.dtype == (out_dtype or torch.bfloat16) and tuple(y.shape) == (m, N)
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"m={m}: bound call differs from the op"
    # a 3-D input and a row-strided view (the op's copy of rows with an unaligned stride)
    x3 = _act(2 * 40).reshape(2, 40, K)
    assert torch.equal(mod(x3).reshape(80, N).view(torch.int16), _op(mod, x3.reshape(80, K)).view(torch.int16))
    xw = _act(64)
    xs = torch.cat([xw, xw[:, :8]], dim=1)[:, :K]          # row stride K + 8 (aligned)
    xu = torch.cat([xw, xw[:, :3]], dim=1)[:, :K]          # row stride K + 3 (copied)
    for xv in (xs, xu):
        assert torch.equal(mod(xv).view(torch.int16), _op(mod, xv.contiguous()).view(torch.int16))


def test_bound_forward_half_stage():
    """in_features % 128 == 64 (the records end in a half stage; no GEMV): the bound call equals the op."""
    from gen_worker_amd import synthetic
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    k = 320
    L = synthetic.w4a4_layer(N, k, 32, seed_offset=9)
    mod = build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                 proj_up=L.proj_up, bias=L.bias, device=DEV)
    assert mod.lane == "fp6" and mod._gemv_max_m == 0 and int(mod.weight_fp6.shape[0]) == 3
    for m in (0, 1, 77, 300):
        x = synthetic.activation(m, k, outlier_frac=0.005, outlier_scale=30.0, seed=13 + m).to(DEV)
        y = mod(x)
        assert mod._bound is not None
        ref = _op(mod, x)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"m={m}"


def test_bound_call_rebinds_on_changes():
    mod = _module(32, True)
    x = _act(200)
    y0 = mod(x)
    b0 = mod._bound
    assert b0 is not None
    assert mod(x) is not None and mod._bound is b0, "a repeat call rebinds"
    # output dtype and activation are part of the binding
    mod.out_dtype = torch.float16
    y1 = mod(x)
    assert y1.dtype == torch.float16 and mod._bound is not b0
    assert torch.equal(y1.view(torch.int16), _op(mod, x).view(torch.int16))
    mod.out_dtype = None
    mod.activation = "gelu_tanh"
    assert torch.equal(mod(x).view(torch.int16), _op(mod, x).view(torch.int16))
    mod.activation = None
    # a bias swapped under the same Parameter (new storage) and a new bias tensor
    with torch.no_grad():
        mod.bias.data = mod.bias.data * 2
    y2 = mod(x)
    assert not torch.equal(y2, y0)
    assert torch.equal(y2.view(torch.int16), _op(mod, x).view(torch.int16))
    mod.bias = torch.nn.Parameter(torch.zeros_like(mod.bias), requires_grad=False)
    assert torch.equal(mod(x).view(torch.int16), _op(mod, x).view(torch.int16))
    # in-place updates keep the storage: the binding stays and reads the new values
    b = mod._bound
    with torch.no_grad():
        mod.bias.fill_(0.5)
    y3 = mod(x)
    assert mod._bound is b
    assert torch.equal(y3.view(torch.int16), _op(mod, x).view(torch.int16))
    # a module move drops the derived buffers and the binding
    mod.to(DEV)
    assert mod._bound is None
    assert torch.equal(mod(x).view(torch.int16), _op(mod, x).view(torch.int16))


def test_in_place_weight_updates_rebuild_the_derived_buffers():
    """Every buffer of a module overwritten in place with another module's values (same storages): the next
    forward rebuilds the fp6 weight records and proj_down's operand orders, and equals the other module bit for
    bit on the fp6 lane and on the small-M GEMV."""
    mod, other = _module(32, True, seed=3), _module(32, True, seed=11)
    xs = [_act(200), _act(3)]
    assert mod._gemv_max_m >= 3
    before = [mod(x) for x in xs]
    with torch.no_grad():
        for name in ("weight", "weight_scale", "smooth_factor", "proj_down", "proj_up", "bias"):
            getattr(mod, name).copy_(getattr(other, name))
    for x, y0 in zip(xs, before):
        y = mod(x)
        assert not torch.equal(y, y0)
        assert torch.equal(y.view(torch.int16), other(x).view(torch.int16)), f"M={x.shape[0]}"


class _Passthrough(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.ops = []

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.ops.append(str(func))
        return func(*args, **(kwargs or {}))


def test_dispatch_mode_takes_the_op():
    mod = _module(32, True)
    x = _act(96)
    ref = mod(x)
    mode = _Passthrough()
    with mode:
        y = mod(x)
    assert any("svdq_forward_fp6" in o for o in mode.ops), mode.ops
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def _w8_module(mode, static, bias_dtype, out_dtype):
    from gen_worker_amd import synthetic
    from gen_worker_amd.w8a8 import build_int8_linear

    L = synthetic.w8a8_layer(N, K, bias=bias_dtype is not None, seed_offset=5)
    b = L.bias.to(bias_dtype) if bias_dtype is not None else None
    s = torch.tensor([[0.04]]) if static else None
    return build_int8_linear(qweight=L.qweight, weight_scale=L.weight_scale, bias=b, compute_dtype=out_dtype,
                             device=DEV, input_scale=s, gemm_mode=mode)


def _w8_op(mod, x):
    cg = torch.ops.cozy_gen_worker
    q, sa = cg.w8a8_quant(x, mod.gemm_mode == "pertensor", mod.input_scale)
    return cg.w8a8_scaled_mm(q, mod.weight, sa, mod.weight_scale, mod.bias, mod.compute_dtype)


@pytest.mark.parametrize("mode,static,bias_dtype,out_dtype", [
    ("rowwise", False, torch.float32, torch.bfloat16),
    ("rowwise", True, torch.bfloat16, torch.float16),
    ("pertensor", False, None, torch.bfloat16),
    ("pertensor", True, torch.float16, torch.float16),
])
def test_w8a8_bound_forward_equals_the_ops(mode, static, bias_dtype, out_dtype):
    mod = _w8_module(mode, static, bias_dtype, out_dtype)
    for m in (0, 1, 77, 300):
        x = _act(m, seed=11)
        y = mod(x)
        assert mod._bound is not None, "the eager forward did not take the bound call"
        ref = _w8_op(mod, x)
        torch.cuda.synchronize()
        assert y.dtype == out_dtype and tuple(y.shape) == (m, N)
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"m={m}: bound call differs from the ops"


def test_w8a8_bound_call_rebinds_on_changes():
    mod = _w8_module("rowwise", False, torch.float32, torch.bfloat16)
    x = _act(150, seed=11)
    mod(x)
    b0 = mod._bound
    mod.gemm_mode = "pertensor"
    y = mod(x)
    assert mod._bound is not b0
    assert torch.equal(y.view(torch.int16), _w8_op(mod, x).view(torch.int16))
    with torch.no_grad():
        mod.weight_scale.data = mod.weight_scale.data * 0.5
    y2 = mod(x)
    assert torch.equal(y2.view(torch.int16), _w8_op(mod, x).view(torch.int16))
    mod.to(DEV)
    assert mod._bound is None
