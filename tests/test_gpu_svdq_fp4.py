"""GPU tests of the svdq fp4 packaging's blockwise module (``SvdqFp4Linear``) against the oracle's restatement of
the reference's forward (``_SvdqLinear.forward``, ``models/svdq_native.py:140-156``), at a small shape with
every option, at the QKV shape on a row sample (the dynamic scale s2 is the whole call's), and through the
artifact loader with a fused projection split."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits16, check_output
from oracle import nvfp4_oracle as F4
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


def _f(t):
    return None if t is None else t.float().cpu().numpy()


def _oracle(dec, x, s2=None):
    xf = O.bf16_bits_to_f32(bits16(x))
    return F4.svdq_fp4_linear(xf, _f(dec.smooth_factor), F4.pack_e2m1(dec.codes.numpy()),
                              dec.scales.view(torch.uint8).numpy(), dec.second.numpy(), _f(dec.proj_down),
                              _f(dec.proj_up), _f(dec.bias), s2=s2)


@pytest.mark.parametrize("per_channel,smooth,rank,bias", [(True, True, 32, True), (False, False, 0, False),
                                                          (False, True, 16, True), (True, False, 32, False)])
def test_svdq_fp4_module_matches_the_oracle(per_channel, smooth, rank, bias):
    from gen_worker_amd import svdq_fp4 as S
    from gen_worker_amd import synthetic

    n, k, m = 256, 512, 77
    L = synthetic.svdq_fp4_layer(n, k, rank, per_channel=per_channel, smooth=smooth, bias=bias, seed_offset=9)
    dec = S.decode_fp4_linear(L.stored, n, k)
    mod = S.build_fp4_module(dec, device=DEV, mode="blockwise")
    assert isinstance(mod, S.SvdqFp4Linear) and mod.per_channel_scale == per_channel
    x = synthetic.activation(m, k, outlier_frac=0.01, outlier_scale=20.0, seed=61).to(DEV)
    y = mod(x)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, n)
    check_output(y, _oracle(dec, x), what=f"svdq fp4 [{n}, {k}] pc={per_channel} smooth={smooth} r={rank}")
    # a leading batch shape is kept
    y3 = mod(x.reshape(7, 11, k))
    assert tuple(y3.shape) == (7, 11, n) and torch.equal(y3.reshape(m, n).view(torch.int16), y.view(torch.int16))


def test_svdq_fp4_qkv_row_sample():
    from gen_worker_amd import svdq_fp4 as S
    from gen_worker_amd import synthetic

    n, k, r, m = 9216, 3072, 32, 1024
    L = synthetic.svdq_fp4_layer(n, k, r, per_channel=True, seed_offset=13)
    dec = S.decode_fp4_linear(L.stored, n, k)
    mod = S.build_fp4_module(dec, device=DEV, mode="blockwise")
    x = synthetic.activation(m, k, outlier_frac=0.005, outlier_scale=30.0, seed=1000 + m).to(DEV)
    y, y2 = mod(x), mod(x)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.equal(y.view(torch.int16), y2.view(torch.int16)), "not deterministic"
    xs = F4.bf16_round(O.bf16_bits_to_f32(bits16(x)) / _f(dec.smooth_factor).reshape(1, -1))
    s2 = F4.dynamic_s2(xs)                                   # the whole call's scale, as the module takes it
    rows = np.unique(np.r_[0:4, 255:258, 511:514, m - 4:m])
    check_output(y[rows], _oracle(dec, x[rows], s2=s2), what="svdq fp4 QKV M=1024 rows")
    # the dense fold computes the same linear without the activation's 4-bit rounding: close, not equal
    dense = S.build_fp4_module(dec, device=DEV, mode="dense")
    yd = dense(x).float()
    rel = float((y.float() - yd).norm() / yd.norm())
    print(f"blockwise vs dense fold: rel_fro {rel:.3e}")
    assert rel < 0.2, rel


def test_load_fp4_artifact_blockwise(tmp_path):
    import torch.nn as nn

    from gen_worker_amd import svdq_artifact as A
    from gen_worker_amd import svdq_checkpoint as C
    from gen_worker_amd import svdq_fp4 as S
    from gen_worker_amd import synthetic
    from test_svdq_fp4 import _fp4_snapshot, _skeleton

    d = 256
    qkv, out = _fp4_snapshot(tmp_path, d, 32)
    model = _skeleton(d)
    counts = A.load_svdq_artifact(tmp_path / "snap", model, device=DEV, lane="dense", fp4_mode="blockwise")
    assert counts["blockwise"] == 4 and counts["dense"] == 0 and counts["fp4_mode"] == "blockwise"
    attn = model.blocks[0].attn
    parts = C.split_decoded(S.decode_fp4_linear(qkv.stored, 3 * d, d), (d, d, d))
    x = synthetic.activation(40, d, outlier_frac=0.01, outlier_scale=20.0, seed=62).to(DEV)
    for name, mod, part in zip("qkv", (attn.to_q, attn.to_k, attn.to_v), parts):
        assert isinstance(mod, S.SvdqFp4Linear)
        check_output(mod(x), _oracle(part, x), what=f"loaded to_{name}")
    o = attn.to_out[0]
    assert isinstance(o, S.SvdqFp4Linear) and not o.per_channel_scale and not isinstance(o, nn.Linear)
    check_output(o(x), _oracle(S.decode_fp4_linear(out.stored, d, d), x), what="loaded to_out")
