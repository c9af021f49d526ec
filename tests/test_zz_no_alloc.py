"""The zero-allocation linear entry point (``gwa_svdq_w4a4_linear_fp6_noalloc``) through the C-ABI.

It runs the same kernels as ``gwa_svdq_w4a4_linear_fp6`` on a static scratch array instead of a caller
workspace, so its outputs must equal that entry point's bit for bit: checked on two calls in a row (the second
with a smaller input, over the scratch contents the first left), plus the oracle on sampled rows, the size limit
(refused before anything is enqueued) and the device's free memory across the calls.
"""

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
    assert torch.cuda.is_available()
    yield


def _module(n, k, r, seed):
    from gen_worker_amd import synthetic
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    L = synthetic.w4a4_layer(n, k, r, seed_offset=seed)
    mod = build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                 proj_up=L.proj_up, bias=L.bias, device=DEV)
    assert mod.lane == "fp6"
    return L, mod


def _args(mod, x, out, gelu=False):
    from gen_worker_amd import _native as nat
    from gen_worker_amd import ops

    m, k = int(x.shape[0]), int(x.shape[1])
    return (nat.ptr(x), k, nat.ptr(mod.smooth_factor), None, nat.ptr(mod.proj_down_op6) if mod.rank else None,
            mod.rank, nat.ptr(mod.weight_fp6), ops.readable_bytes(mod.weight_fp6), nat.ptr(mod.second),
            int(mod.second.numel()),
            nat.ptr(mod.proj_up) if mod.rank else None, nat.ptr(mod.bias), nat.ptr(out), nat.DT_BF16,
            nat.EPI_GELU_TANH if gelu else 0, m, mod.out_features, k)


def _with_workspace(mod, x, gelu=False):
    from gen_worker_amd import _native as nat
    from gen_worker_amd import ops

    out = torch.empty(int(x.shape[0]), mod.out_features, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(ops.linear_fp6_workspace_bytes(int(x.shape[0]), int(x.shape[1]), mod.rank), dtype=torch.uint8,
                     device=DEV)
    nat.call("gwa_svdq_w4a4_linear_fp6", *_args(mod, x, out, gelu), nat.ptr(ws), int(ws.numel()), nat.stream_of(x))
    return out


def _no_alloc(mod, x, out, gelu=False):
    from gen_worker_amd import _native as nat

    nat.call("gwa_svdq_w4a4_linear_fp6_noalloc", *_args(mod, x, out, gelu), nat.stream_of(x))
    return out


def test_no_alloc_matches_workspace_entry_point():
    from gen_worker_amd import synthetic

    La, big = _module(3072, 3072, 32, seed=0)       # config 1's layer
    Lb, small = _module(512, 1024, 16, seed=7)
    xa = synthetic.activation(4608, 3072, outlier_frac=0.005, outlier_scale=30.0).to(DEV)
    xb = synthetic.activation(77, 1024, outlier_frac=0.01, outlier_scale=20.0, seed=9).to(DEV)
    want_a = _with_workspace(big, xa)
    want_b = _with_workspace(small, xb, gelu=True)
    ya = torch.empty_like(want_a)
    yb = torch.empty_like(want_b)
    _no_alloc(small, xb, torch.empty_like(want_b))   # first call on this device: the scratch address lookup
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    _no_alloc(big, xa, ya)                          # two calls in a row, the second smaller
    _no_alloc(small, xb, yb, gelu=True)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"device free memory changed across the no-alloc calls: {free0} -> {free1}"
    assert torch.equal(ya.view(torch.int16), want_a.view(torch.int16)), "first call differs from the workspace path"
    assert torch.equal(yb.view(torch.int16), want_b.view(torch.int16)), "second call differs from the workspace path"
    rows = np.r_[0:24, 4608 - 24:4608]
    ref = O.w4a4_linear(bits16(xa[rows]), bits16(La.smooth), La.qweight.numpy(), La.wscales.numpy(),
                        bits16(La.proj_down), bits16(La.proj_up), bits16(La.bias))
    check_output(ya[rows], ref, what="no-alloc config-1 rows")
    ref_b = O.w4a4_linear(bits16(xb), bits16(Lb.smooth), Lb.qweight.numpy(), Lb.wscales.numpy(),
                          bits16(Lb.proj_down), bits16(Lb.proj_up), bits16(Lb.bias), gelu=True)
    check_output(yb, ref_b, what="no-alloc small layer")


def test_no_alloc_refuses_shapes_beyond_its_scratch():
    from gen_worker_amd import _native as nat
    from gen_worker_amd import ops

    lib = nat.load()
    cap = int(lib.gwa_svdq_w4a4_linear_fp6_noalloc_scratch_bytes())
    assert cap == 128 << 20
    m = 1
    while ops.linear_fp6_workspace_bytes(m * 2, 3072, 32) <= cap:
        m *= 2
    lo, hi = m, m * 2
    while hi - lo > 1:
        mid = (lo + hi) // 2
        lo, hi = (mid, hi) if ops.linear_fp6_workspace_bytes(mid, 3072, 32) <= cap else (lo, mid)
    too_big = hi
    dummy = 256   # never dereferenced: the size check comes first
    rc = lib.gwa_svdq_w4a4_linear_fp6_noalloc(dummy, 3072, None, None, dummy, 32, dummy, 1 << 30, None, 0, dummy, None,
                                              dummy, nat.DT_BF16, 0, too_big, 3072, 3072, None)
    assert rc == 1 and "static scratch holds" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_w4a4_linear_fp6_noalloc(None, 3072, None, None, None, 0, None, 0, None, 0, None, None, None,
                                              nat.DT_BF16, 0, 0, 3072, 3072, None)
    assert rc == 0   # M = 0: nothing to do
