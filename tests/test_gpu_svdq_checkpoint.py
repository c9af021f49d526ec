"""GPU: an int4 svdq checkpoint (nunchaku packaging, written to a safetensors file by the oracle's
packers) loaded into a module skeleton: the fused to_qkv split across to_q / to_k / to_v, the other
linears swapped for SvdqW4A4Linear, an AWQ W4A16 modulation layer with six adaLN splits, a plain tensor
copied; every swapped module against the dequantize-then-matmul oracle on the logical tensors."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from helpers import bits16, check_output
from oracle import svdq_oracle as O
from test_svdq_checkpoint import synthetic_int4_layer

from gen_worker_amd import awq
from gen_worker_amd import svdq_checkpoint as C
from gen_worker_amd.svdq import SvdqW4A4Linear

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 256


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.to_q, self.to_k, self.to_v = nn.Linear(D, D), nn.Linear(D, D), nn.Linear(D, D)
        self.to_out = nn.ModuleList([nn.Linear(D, D)])


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn = _Attn()
        self.ff_out = nn.Linear(2 * D, D)
        self.norm1 = nn.Module()
        self.norm1.linear = nn.Linear(D, 6 * D)
        self.register_buffer("scale_table", torch.zeros(4, D))



def test_load_int4_checkpoint(tmp_path):
    from safetensors.torch import save_file

    qkv_l, qkv_s = synthetic_int4_layer(3 * D, D, 32, seed=11)
    out_l, out_s = synthetic_int4_layer(D, D, 16, seed=12, second="channel")
    ff_l, ff_s = synthetic_int4_layer(D, 2 * D, 32, seed=13)
    g = torch.Generator().manual_seed(14)
    w_mod, b_mod = torch.randn(6 * D, D, generator=g) * 0.02, torch.randn(6 * D, generator=g) * 0.02
    awq_t = awq.encode_awq_linear(w_mod, b_mod, adanorm_splits=6)
    table = torch.randn(4, D, generator=g)
    tensors = {}
    for prefix, st in (("blocks.0.attn.to_qkv", qkv_s), ("blocks.0.attn.to_out.0", out_s), ("blocks.0.ff_out", ff_s)):
        tensors.update({f"{prefix}.{k}": v.contiguous() for k, v in st.items()})
    tensors.update({f"blocks.0.norm1.linear.{k}": v.contiguous() for k, v in awq_t.items()})
    tensors["blocks.0.scale_table"] = table
    path = tmp_path / "svdq_int4.safetensors"
    save_file(tensors, str(path))

    model = nn.Module()
    model.blocks = nn.ModuleList([_Block()])
    counts = C.load_svdq_int4_checkpoint(path, model, adanorm_splits={"blocks.0.norm1.linear": 6}, device=DEV,
                                         lane="int4")
    assert counts["int4_prefixes"] == 3 and counts["linears"] == 5 and counts["int4"] == 5
    assert counts["awq"] == 1 and counts["plain"] == 1
    blk = model.blocks[0]
    assert torch.equal(blk.scale_table.cpu(), table)
    gx = torch.Generator().manual_seed(15)
    for name, mod, logical, rows, k in (("to_q", blk.attn.to_q, qkv_l, slice(0, D), D),
                                        ("to_k", blk.attn.to_k, qkv_l, slice(D, 2 * D), D),
                                        ("to_v", blk.attn.to_v, qkv_l, slice(2 * D, 3 * D), D),
                                        ("to_out", blk.attn.to_out[0], out_l, slice(0, D), D),
                                        ("ff_out", blk.ff_out, ff_l, slice(0, D), 2 * D)):
        assert isinstance(mod, SvdqW4A4Linear), name
        x = torch.randn(77, k, generator=gx).to(torch.bfloat16)
        with torch.no_grad():
            y = mod(x.to(DEV))
        codes = logical["codes"][rows]
        packed = (codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)
        second = logical["second"][rows] if "second" in logical else None
        ref = O.w4a4_linear(bits16(x), bits16(logical["smooth"]), packed, logical["scales"][rows],
                            bits16(logical["down"]), bits16(logical["up"][rows]), bits16(logical["bias"][rows]),
                            second=second)
        check_output(y, ref, what=f"checkpoint {name}")
    # the modulation layer: packed AWQ against the decoded bf16 Linear (rows and bias offsets undone)
    lin = awq.decode_awq_linear(awq_t, 6 * D, D, adanorm_splits=6, device=DEV)
    x = torch.randn(1, D, generator=gx).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        y, yl = blk.norm1.linear(x).float(), lin(x).float()
    assert ((y - yl).norm() / yl.norm()).item() <= 5e-3


@pytest.mark.parametrize("scheme", ["int8", "fp8_e4m3"])
def test_load_artifact_quantized_lowrank(tmp_path, scheme):
    """A snapshot whose svdq-int4 artifact (detected by its metadata in transformer/) stores the low-rank
    branch as int8 / fp8 with block scales: routed onto the int4 lane, each swapped module against the oracle
    on the dequantized factors."""
    import json

    from safetensors.torch import save_file

    from gen_worker_amd import svdq_artifact as SA
    from test_svdq_artifact import _quantized_layer

    logical, stored, down, up = _quantized_layer(3 * D, D, 32, 31, scheme)
    tensors = {f"blocks.0.attn.to_qkv.{k}": v.contiguous() for k, v in stored.items()}
    meta = {"model_class": "NunchakuFluxTransformer2DModel", "lowrank_quant": scheme,
            "quantization_config": json.dumps({"method": "svdquant", "weight": {"dtype": "int4"}, "rank": 32})}
    (tmp_path / "transformer").mkdir()
    save_file(tensors, str(tmp_path / "transformer" / "svdq.safetensors"), metadata=meta)
    model = nn.Module()
    model.blocks = nn.ModuleList([_Block()])
    counts = SA.load_svdq_artifact(tmp_path, model, device=DEV, lane="int4")
    assert counts["int4"] == 3 and counts["artifact"].lowrank_quant == scheme
    blk = model.blocks[0]
    gx = torch.Generator().manual_seed(33)
    for i, mod in enumerate((blk.attn.to_q, blk.attn.to_k, blk.attn.to_v)):
        assert isinstance(mod, SvdqW4A4Linear)
        rows = slice(i * D, (i + 1) * D)
        x = torch.randn(65, D, generator=gx).to(torch.bfloat16)
        with torch.no_grad():
            y = mod(x.to(DEV))
        codes = logical["codes"][rows]
        packed = (codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)
        ref = O.w4a4_linear(bits16(x), bits16(logical["smooth"]), packed, logical["scales"][rows], bits16(down),
                            bits16(up[rows]), bits16(logical["bias"][rows]))
        check_output(y, ref, what=f"quantized low-rank ({scheme}) part {i}")
