"""GPU tests of the one-call fp6-lane linear (``gwa_svdq_w4a4_linear_fp6`` / ``svdq_forward_fp6``), the
operand-record slack contract at the op boundary, and the module's re-derivation of its records after moves.

The one-call path runs the same kernels as ``svdq_quant_fp6`` followed by ``svdq_w4a4_linear_fp6``, so its
output must equal theirs bit for bit; both are checked against the oracle's dequantize-then-matmul.
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


def _layer(n, k, r, seed=0):
    from gen_worker_amd import synthetic

    return synthetic.w4a4_layer(n, k, r, seed_offset=seed)


def _module(L, activation=None, out_dtype=None):
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    return build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth,
                                  proj_down=L.proj_down, proj_up=L.proj_up, bias=L.bias,
                                  activation=activation, out_dtype=out_dtype, device=DEV)


def _two_op(mod, x, out_dtype, gelu):
    ops = torch.ops.cozy_gen_worker
    q6, la = ops.svdq_quant_fp6(x, mod.smooth_factor, None, mod.proj_down_op6 if mod.rank else None)
    return ops.svdq_w4a4_linear_fp6(q6, mod.weight_fp6, None, mod.second, la if mod.rank else None, mod.proj_up,
                                    mod.bias, out_dtype, gelu)


@pytest.mark.parametrize("m,n,k,r,gelu,odt", [
    (77, 256, 512, 32, False, torch.bfloat16),
    (1, 128, 128, 16, False, torch.bfloat16),
    (300, 384, 768, 0, True, torch.float16),
    (513, 640, 1024, 64, True, torch.bfloat16),
    (4608, 3072, 3072, 32, False, torch.bfloat16),
    (4096, 3072, 64, 32, False, torch.bfloat16),    # K % 128 == 64: half stages (Flux's x_embedder)
    (129, 272, 320, 16, True, torch.float16),
])
def test_forward_fp6_equals_two_op_path(m, n, k, r, gelu, odt):
    from gen_worker_amd import synthetic

    L = _layer(n, k, r)
    mod = _module(L, "gelu_tanh" if gelu else None, odt)
    assert mod.lane == "fp6"
    x = synthetic.activation(m, k, outlier_frac=0.005, outlier_scale=30.0).to(DEV)
    y1 = mod(x)
    y2 = _two_op(mod, x, odt, gelu)
    torch.cuda.synchronize()
    assert y1.dtype == odt and tuple(y1.shape) == (m, n)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), f"one-call path differs at {m}x{n}x{k} r{r}"
    rows = np.unique(np.clip(np.r_[0:min(m, 40), m - 40:m], 0, m - 1))
    ref = O.w4a4_linear(bits16(x[rows]), bits16(L.smooth), L.qweight.numpy(), L.wscales.numpy(),
                        bits16(L.proj_down) if r else None, bits16(L.proj_up) if r else None, bits16(L.bias),
                        gelu=gelu)
    check_output(y1[rows], ref, what=f"forward_fp6 {m}x{n}x{k} r{r}")


def test_linear_entry_point_workspace_contract():
    """The C-ABI entry point itself: exactly the reported workspace works (and equals the op), one byte less is
    refused before anything is enqueued, a misaligned workspace is refused."""
    from gen_worker_amd import _native as nat
    from gen_worker_amd import ops, synthetic

    m, n, k, r = 200, 256, 384, 32
    L = _layer(n, k, r, seed=3)
    mod = _module(L)
    x = synthetic.activation(m, k, outlier_frac=0.01, outlier_scale=20.0).to(DEV)
    want = mod(x)
    need = ops.linear_fp6_workspace_bytes(m, k, r)
    assert need > m * (k // 128) * nat.FP6_REC + ops.RECORD_SLACK
    ws = torch.empty(need + 256, dtype=torch.uint8, device=DEV)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    args = lambda w, nbytes: (nat.ptr(x), k, nat.ptr(mod.smooth_factor), None, nat.ptr(mod.proj_down_op6), r,  # noqa: E731
                              nat.ptr(mod.weight_fp6), ops.readable_bytes(mod.weight_fp6), nat.ptr(mod.second), 1,
                              nat.ptr(mod.proj_up),
                              nat.ptr(mod.bias), nat.ptr(out), nat.DT_BF16, 0, m, n, k, w, nbytes,
                              nat.stream_of(x))
    nat.call("gwa_svdq_w4a4_linear_fp6", *args(ws.data_ptr(), need))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    with pytest.raises(nat.NativeError, match="workspace of"):
        nat.call("gwa_svdq_w4a4_linear_fp6", *args(ws.data_ptr(), need - 1))
    with pytest.raises(nat.NativeError, match="256-byte aligned"):
        nat.call("gwa_svdq_w4a4_linear_fp6", *args(ws.data_ptr() + 16, need))


def test_record_slack_refused_at_the_op():
    """A record tensor without the 1 KB of readable storage the GEMM's copies may reach is refused before launch."""
    from gen_worker_amd import ops
    from gen_worker_amd.ops import SvdqOpError

    mod = _module(_layer(256, 256, 16))
    x = torch.randn(64, 256, device=DEV).to(torch.bfloat16)
    q6, la = torch.ops.cozy_gen_worker.svdq_quant_fp6(x, mod.smooth_factor, None, mod.proj_down_op6)
    assert ops.record_slack_bytes(q6) >= ops.RECORD_SLACK
    bare = q6.clone()   # exact-size storage
    assert ops.record_slack_bytes(bare) == 0
    with pytest.raises(SvdqOpError, match="readable bytes past its last record"):
        torch.ops.cozy_gen_worker.svdq_w4a4_linear_fp6(bare, mod.weight_fp6, None, mod.second, la, mod.proj_up,
                                                       mod.bias, torch.bfloat16, False)
    with pytest.raises(SvdqOpError, match="weight_fp6"):
        torch.ops.cozy_gen_worker.svdq_w4a4_linear_fp6(q6, mod.weight_fp6.clone(), None, mod.second, la,
                                                       mod.proj_up, mod.bias, torch.bfloat16, False)
    with pytest.raises(SvdqOpError, match="weight_fp6"):
        torch.ops.cozy_gen_worker.svdq_forward_fp6(x, mod.smooth_factor, None, mod.proj_down_op6,
                                                   mod.weight_fp6.clone(), mod.second, mod.proj_up, mod.bias,
                                                   torch.bfloat16, False)


def test_module_moves_rederive_records():
    """``.cpu().cuda()`` (and ``.to``) copy buffers without slack: the module drops its derived records on a move
    and rebuilds them with slack on the next forward, which equals the forward before the move."""
    from gen_worker_amd import ops, synthetic

    mod = _module(_layer(384, 512, 32, seed=5))
    x = synthetic.activation(96, 512, outlier_frac=0.01, outlier_scale=20.0).to(DEV)
    before = mod(x)
    mod = mod.cpu()
    assert mod.weight_fp6 is None and mod.proj_down_op6 is None and mod.proj_down_op is None
    mod = mod.cuda()
    assert mod.weight_fp6 is None
    after = mod(x)
    torch.cuda.synchronize()
    assert mod.weight_fp6 is not None and ops.record_slack_bytes(mod.weight_fp6) >= ops.RECORD_SLACK
    assert torch.equal(before.view(torch.int16), after.view(torch.int16))
