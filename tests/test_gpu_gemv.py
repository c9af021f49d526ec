"""The small-M W4A4 path (``gwa_svdq_w4a4_linear_gemv`` / ``cozy_gen_worker::svdq_forward_gemv``; the module
takes it for up to ``gemv_max_m`` tokens): the int4 weight streamed once, rows quantized with kernel 1's
quantizer, kernel 1's la partial slots summed in order.

Pinned three ways: against the float64 oracle chain (``oracle.svdq_oracle.w4a4_linear``) to the per-linear
bar of every W4A4 output; bit for bit (bf16 outputs) against the fp6 GEMM lane when there is no low-rank
branch (same codes and scales, same group order acc = fma(P_g, sx_g * sw_g, acc), same epilogue), which
fails on any wrong code, scale, group product or ordering; and within one bf16 step of it with the low-rank
branch (whose sum the GEMM takes through a bf16 MFMA). Shapes: the DiT's modulation linears (one token, K=3072 -> 18432 and
9216), every M up to the limit, the largest K, ragged N, per-channel second, GELU, fp16 out, no smoothing."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits16, check_output
from oracle import svdq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native

    _native.load()
    yield


def _layer(n, k, rank, *, smooth=True, bias=True, per_channel=False, gelu=False, seed=0):
    from gen_worker_amd import synthetic
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    L = synthetic.w4a4_layer(n, k, rank, smooth=smooth, bias=bias, seed_offset=seed)
    sec = None
    if per_channel:
        sec = (0.5 + torch.rand(n, generator=torch.Generator().manual_seed(seed + 99))).float()
    mod = build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                 proj_up=L.proj_up, bias=L.bias, second=sec, device=DEV,
                                 activation="gelu_tanh" if gelu else None)
    mod._ensure_derived()
    return L, mod


def _gemv(mod, x, out_dtype=torch.bfloat16, second=None):
    cg = torch.ops.cozy_gen_worker
    return cg.svdq_forward_gemv(x, mod.smooth_factor, None, mod.proj_down_op6 if mod.rank else None, mod.weight,
                                mod.weight_scale, mod.second if second is None else second, mod.proj_up,
                                mod.bias, out_dtype, mod.activation == "gelu_tanh")


def _gemm(mod, x, out_dtype=torch.bfloat16):
    cg = torch.ops.cozy_gen_worker
    return cg.svdq_forward_fp6(x, mod.smooth_factor, None, mod.proj_down_op6 if mod.rank else None, mod.weight_fp6,
                               mod.second, mod.proj_up, mod.bias, out_dtype, mod.activation == "gelu_tanh")


def _oracle(L, mod, x):
    sec = mod.second.float().cpu().numpy() if mod.second is not None else None
    return O.w4a4_linear(bits16(x.cpu()), bits16(L.smooth) if L.smooth is not None else None, L.qweight.numpy(),
                         L.wscales.numpy(), bits16(L.proj_down) if L.proj_down is not None else None,
                         bits16(L.proj_up) if L.proj_up is not None else None,
                         bits16(L.bias) if L.bias is not None else None, second=sec,
                         gelu=mod.activation == "gelu_tanh")


def _x(m, k, seed=0):
    from gen_worker_amd import synthetic

    return synthetic.activation(m, k, outlier_frac=0.005, outlier_scale=30.0, seed=seed).to(DEV)


def test_limits():
    from gen_worker_amd import ops

    assert ops.gemv_max_m(3072, 32) == 8 and ops.gemv_max_m(3072, 0) == 8
    assert ops.gemv_max_m(8192, 32) == 4 and ops.gemv_max_m(12288, 32) == 0 and ops.gemv_max_m(192, 32) == 0
    _, mod = _layer(256, 3072, 32)
    assert mod._gemv_max_m == 8
    with pytest.raises(Exception, match="small-M path"):
        _gemv(mod, _x(9, 3072))


@pytest.mark.parametrize("n", [18432, 9216])
def test_modulation_shapes_match_oracle(n):
    L, mod = _layer(n, 3072, 32, seed=n)
    x = _x(1, 3072, seed=1)
    y = _gemv(mod, x)
    check_output(y, _oracle(L, mod, x), what=f"gemv 1x{n}x3072")
    yg = _gemm(mod, x)
    diff = (y != yg)
    assert diff.float().mean().item() < 0.02   # only the low-rank sum's rounding differs
    d = (y.float() - yg.float()).abs()[diff]
    if d.numel():
        assert (d <= 2.0 ** -7 * y.float().abs()[diff].clamp_min(2.0 ** -8)).all()


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
def test_rank0_bit_identical_to_gemm_lane(m):
    for gelu, per_channel, smooth in ((False, False, True), (True, True, True), (False, True, False)):
        L, mod = _layer(384, 3072, 0, per_channel=per_channel, gelu=gelu, smooth=smooth, seed=m)
        x = _x(m, 3072, seed=m)
        y = _gemv(mod, x)
        assert torch.equal(y, _gemm(mod, x)), (m, gelu, per_channel, smooth)
        check_output(y, _oracle(L, mod, x), what=f"gemv rank0 m={m}")
        # fp16 keeps 3 more bits: the GEMM's compiled epilogue forms acc * mult + bias as one fma for most of a
        # lane's elements and as a multiply and an add for the rest, which moves an fp16 rounding by one step
        # in rare elements (1 of 3072 at m = 8 with GELU and per-channel scales)
        y16, g16 = _gemv(mod, x, torch.float16), _gemm(mod, x, torch.float16)
        d = y16 != g16
        assert d.float().mean().item() < 2e-3, (m, gelu, per_channel, smooth)
        assert bool(((y16.float() - g16.float()).abs()[d] <= 2.0 ** -10 * g16.float().abs()[d]).all())


def test_plain_lds_layout_bit_identical_to_gemm_lane():
    """K = 6144 with 6 tokens and rank 0: the padded LDS layout would pass 64 KB, so the kernel keeps the plain
    strides (8 and G dwords); the result is the fp6 GEMM lane's bit for bit, as with the padded layout."""
    from gen_worker_amd import ops

    assert ops.gemv_max_m(6144, 0) >= 6
    L, mod = _layer(64, 6144, 0, per_channel=True, gelu=False, smooth=True, seed=61)
    x = _x(6, 6144, seed=61)
    y = _gemv(mod, x)
    assert torch.equal(y, _gemm(mod, x))
    check_output(y, _oracle(L, mod, x), what="gemv plain layout 6x64x6144 r0")


@pytest.mark.parametrize("m,k,n,rank", [(4, 8192, 160, 32), (1, 128, 16, 16), (7, 1024, 48, 64),
                                        (2, 3072, 272, 128)])
def test_shapes_match_oracle(m, k, n, rank):
    L, mod = _layer(n, k, rank, per_channel=True, gelu=rank == 64, seed=k + n)
    x = _x(m, k, seed=k)
    y = _gemv(mod, x)
    check_output(y, _oracle(L, mod, x), what=f"gemv {m}x{n}x{k} r{rank}")


def test_module_routes_small_m_and_graph_replays():
    L, mod = _layer(6144, 3072, 32, seed=5)
    x = _x(1, 3072, seed=5)
    with torch.no_grad():
        y = mod(x)
    assert torch.equal(y, _gemv(mod, x))       # the module's one-token forward is the GEMV
    x16 = _x(16, 3072, seed=6)
    with torch.no_grad():
        assert torch.equal(mod(x16), _gemm(mod, x16))   # above the limit: the GEMM lane
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            yg = mod(x)
    torch.cuda.synchronize()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y)
        with torch.no_grad():
            mod(x16)
        torch.cuda.synchronize()
