"""CPU tests: recognising svdq checkpoints in a snapshot by their safetensors ``__metadata__``, the
servability refusals, routing a detected int4 artifact into a model (dense lane on the CPU), and the
quantized low-rank branch (int8 / fp8 e4m3 factors with per-32 block scales)."""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest
import torch
import torch.nn as nn
from safetensors.torch import save_file

from oracle import svdq_oracle as O
from test_svdq_checkpoint import synthetic_int4_layer

from gen_worker_amd import svdq_artifact as A
from gen_worker_amd import svdq_checkpoint as C


def _qc(dtype="int4", rank=32, as_string=True):
    qc = {"method": "svdquant", "weight": {"dtype": dtype}, "rank": rank}
    return json.dumps(qc) if as_string else qc


def _write(path, meta, tensors=None):
    path.parent.mkdir(parents=True, exist_ok=True)
    save_file(tensors or {"x": torch.zeros(2)}, str(path), metadata=meta)
    return path


def test_metadata_reader(tmp_path):
    p = _write(tmp_path / "a.safetensors", {"model_class": "NunchakuFluxTransformer2DModel", "k": "v"})
    assert A.read_safetensors_metadata(p) == {"model_class": "NunchakuFluxTransformer2DModel", "k": "v"}
    short = tmp_path / "short.safetensors"
    short.write_bytes(b"\x01\x02")
    assert A.read_safetensors_metadata(short) == {}
    huge = tmp_path / "huge.safetensors"
    huge.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")      # a declared header far past the limit: not read
    assert A.read_safetensors_metadata(huge) == {}
    # the bound is the reference's MAX_HEADER_BYTES (models/safetensors_header.py:11); one byte past it is
    # refused before any read
    assert A.HEADER_LIMIT == 100 * 1024 * 1024
    over = tmp_path / "over.safetensors"
    over.write_bytes(struct.pack("<Q", A.HEADER_LIMIT + 1) + b'{"__metadata__": {"a": "b"}}')
    assert A.read_safetensors_metadata(over) == {}
    assert A.read_safetensors_metadata(tmp_path / "missing.safetensors") == {}


def test_detection_rules(tmp_path):
    meta = {"model_class": "NunchakuQwenImageTransformer2DModel", "quantization_config": _qc("int4", 32)}
    p = _write(tmp_path / "bare.safetensors", meta)
    art = A.artifact_of_file(p)
    assert art.precision == "int4" and art.rank == 32 and art.lowrank_quant is None
    assert art.denoiser_class == "QwenImageTransformer2DModel"
    # the config may also be stored as a JSON object inside the metadata string; fp4 is recognised too
    fp4 = A.artifact_of_file(_write(tmp_path / "fp4.safetensors",
                                    {"model_class": "NunchakuFluxTransformer2DModel",
                                     "quantization_config": _qc("fp4_e2m1_all", 128), "lowrank_quant": "int8"}))
    assert fp4.precision == "fp4" and fp4.rank == 128 and fp4.lowrank_quant == "int8"
    # not svdq: another method, a non-nunchaku class, an unknown weight dtype, no metadata at all
    assert A.artifact_of_file(_write(tmp_path / "m.safetensors", {"model_class": "NunchakuX",
                                                                   "quantization_config": json.dumps(
                                                                       {"method": "awq"})})) is None
    assert A.artifact_of_file(_write(tmp_path / "c.safetensors", {"model_class": "FluxTransformer2DModel",
                                                                   "quantization_config": _qc()})) is None
    assert A.artifact_of_file(_write(tmp_path / "d.safetensors", {"model_class": "NunchakuX",
                                                                   "quantization_config": _qc("int8")})) is None
    assert A.artifact_of_file(_write(tmp_path / "plain.safetensors", {})) is None


def test_detection_in_snapshot_layouts(tmp_path):
    meta = {"model_class": "NunchakuFluxTransformer2DModel", "quantization_config": _qc()}
    snap = tmp_path / "snap"
    _write(snap / "vae" / "v.safetensors", meta)                 # not a denoiser folder: ignored
    _write(snap / "transformer" / "a_plain.safetensors", {})
    want = _write(snap / "transformer" / "b_svdq.safetensors", meta)
    _write(snap / "root_svdq.safetensors", meta)
    art = A.detect_svdq_artifact(snap)
    assert art.file == want and art.component == "transformer"
    # without a denoiser folder the root is searched; a bare file is its own artifact
    root_only = tmp_path / "root_only"
    f = _write(root_only / "model.safetensors", meta)
    assert A.detect_svdq_artifact(root_only).file == f and A.detect_svdq_artifact(root_only).component == ""
    assert A.detect_svdq_artifact(f).file == f
    assert A.detect_svdq_artifact(tmp_path / "nothing") is None
    empty = tmp_path / "empty"
    empty.mkdir()
    assert A.detect_svdq_artifact(empty) is None


def test_servability(tmp_path):
    base = dict(component="", file=tmp_path / "x.safetensors", model_class="NunchakuX", rank=32)
    A.check_svdq_servable(A.SvdqArtifact(precision="int4", lowrank_quant=None, **base))
    A.check_svdq_servable(A.SvdqArtifact(precision="int4", lowrank_quant="fp8_e4m3", **base))
    A.check_svdq_servable(A.SvdqArtifact(precision="fp4", lowrank_quant=None, **base))
    A.check_svdq_servable(A.SvdqArtifact(precision="fp4", lowrank_quant="int8", **base))
    with pytest.raises(A.SvdqPrecisionUnsupported, match="svdq-int2"):
        A.check_svdq_servable(A.SvdqArtifact(precision="int2", lowrank_quant=None, **base))
    with pytest.raises(A.SvdqArtifactError, match="lowrank_quant"):
        A.check_svdq_servable(A.SvdqArtifact(precision="int4", lowrank_quant="int4", **base))
    with pytest.raises(A.SvdqArtifactError, match="no svdq checkpoint"):
        A.load_svdq_artifact(tmp_path, nn.Module(), device="cpu", lane="dense")


# ---------------------------------------------------------------------------
# quantized low-rank branch
# ---------------------------------------------------------------------------

def test_lowrank_dequant_known_answers():
    """Codes times power-of-two block scales are exact in bf16: the decoded factor equals them exactly, and
    each scale applies to its own block of 32 along the blocked dimension."""
    q = torch.arange(-32, 32, dtype=torch.int8).reshape(64, 1).repeat(1, 2)      # [64, 2], blocks along rows
    s = torch.tensor([[0.5, 2.0], [0.25, 4.0]])                                  # [64/32, 2]
    got = C.dequantize_lowrank_factor(q, s, along_rows=True)
    want = q.float() * torch.tensor([0.5] * 32 + [0.25] * 32).reshape(64, 1) * torch.tensor([1.0, 1.0])
    want[:, 1] = q[:, 1].float() * torch.tensor([2.0] * 32 + [4.0] * 32)
    assert got.dtype == torch.bfloat16 and torch.equal(got.float(), want)
    qu = torch.ones(3, 64, dtype=torch.int8)                                      # blocks along columns
    su = torch.tensor([[1.0, 8.0], [2.0, 16.0], [4.0, 32.0]])
    gu = C.dequantize_lowrank_factor(qu, su, along_rows=False)
    assert torch.equal(gu.float(), su.repeat_interleave(32, dim=1))
    with pytest.raises(C.SvdqLayoutError):
        C.dequantize_lowrank_factor(q, s[:1], along_rows=True)


@pytest.mark.parametrize("scheme", ["int8", "fp8_e4m3"])
def test_lowrank_producer_round_trip(scheme):
    """Producer then decoder: within half a code step (int8) / e4m3's relative spacing, plus bf16 rounding;
    the decoder's value is RN_bf16(code * scale), computed independently in float64."""
    g = torch.Generator().manual_seed(3)
    w = torch.randn(96, 64, generator=g) * 0.02
    for along_rows in (True, False):
        q, s = C.quantize_lowrank_factor(w, scheme, along_rows=along_rows)
        assert q.dtype == C.LOWRANK_SCHEMES[scheme] and s.dtype == torch.float32
        d = C.dequantize_lowrank_factor(q, s, along_rows=along_rows)
        per = s.repeat_interleave(32, dim=0 if along_rows else 1).double()
        exact = q.double() * per
        want = O.bf16_bits_to_f32(O.f32_to_bf16_bits(exact.float().numpy()))
        assert np.array_equal(d.float().numpy(), want)
        # int8: half a code step; e4m3 (3 mantissa bits): half an ulp of the scaled value, or half the
        # subnormal spacing 2^-9 times the scale; then the bf16 rounding of the result
        quant_err = 0.5 * per if scheme == "int8" else w.abs().double() * 2.0 ** -4 + per * 2.0 ** -10
        bound = quant_err + w.abs().double() * 2.0 ** -8 + 1e-12
        assert bool(((d.double() - w.double()).abs() <= bound).all())


def _quantized_layer(n, k, rank, seed, scheme):
    logical, stored = synthetic_int4_layer(n, k, rank, seed)
    qd, sd = C.quantize_lowrank_factor(logical["down"], scheme, along_rows=True)
    qu, su = C.quantize_lowrank_factor(logical["up"], scheme, along_rows=False)
    stored = dict(stored, proj_down=qd, proj_up=qu, proj_down_scale=sd, proj_up_scale=su)
    down = C.dequantize_lowrank_factor(qd, sd, along_rows=True)
    up = C.dequantize_lowrank_factor(qu, su, along_rows=False)
    return logical, stored, down, up


@pytest.mark.parametrize("scheme", ["int8", "fp8_e4m3"])
def test_decode_quantized_lowrank_branch(scheme):
    logical, stored, down, up = _quantized_layer(256, 384, 32, 9, scheme)
    dec = C.decode_int4_linear(stored, 256, 384, lowrank_quant=scheme)
    assert dec.rank == 32 and torch.equal(dec.proj_down, down) and torch.equal(dec.proj_up, up)
    assert np.array_equal(dec.codes.numpy(), logical["codes"])
    # undeclared means bf16 (the reference's default): quantized factors are refused; None decodes by dtype
    with pytest.raises(C.SvdqLayoutError, match="declares"):
        C.decode_int4_linear(stored, 256, 384)
    assert torch.equal(C.decode_int4_linear(stored, 256, 384, lowrank_quant=None).proj_down, down)
    other = "int8" if scheme != "int8" else "fp8_e4m3"
    with pytest.raises(C.SvdqLayoutError, match="declares"):
        C.decode_int4_linear(stored, 256, 384, lowrank_quant=other)
    with pytest.raises(C.SvdqLayoutError, match="proj_up_scale"):
        C.decode_int4_linear({k_: v for k_, v in stored.items() if k_ != "proj_up_scale"}, 256, 384,
                             lowrank_quant=scheme)
    with pytest.raises(C.SvdqLayoutError, match="one scheme"):
        C.decode_int4_linear(dict(stored, proj_up=up), 256, 384, lowrank_quant=scheme)
    _, plain = synthetic_int4_layer(256, 384, 32, 9)
    with pytest.raises(C.SvdqLayoutError, match="not stored quantized"):
        C.decode_int4_linear(dict(plain, proj_down_scale=stored["proj_down_scale"]), 256, 384)


def test_load_artifact_dense_lane(tmp_path):
    """A snapshot with a quantized-low-rank int4 artifact in transformer/, routed into a skeleton in the dense
    lane: the fused projection split, each Linear the fold of its decoded part."""
    d = 128
    _, qkv, qdown, qup = _quantized_layer(3 * d, d, 32, 21, "int8")
    tensors = {f"blocks.0.attn.to_qkv.{k}": v.contiguous() for k, v in qkv.items()}
    tensors["blocks.0.scale_table"] = torch.arange(4.0)
    meta = {"model_class": "NunchakuQwenImageTransformer2DModel", "quantization_config": _qc("int4", 32),
            "lowrank_quant": "int8"}
    _write(tmp_path / "snap" / "transformer" / "svdq.safetensors", meta, tensors)

    class _Attn(nn.Module):
        def __init__(self):
            super().__init__()
            self.to_q, self.to_k, self.to_v = nn.Linear(d, d), nn.Linear(d, d), nn.Linear(d, d)

    class _Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = _Attn()
            self.register_buffer("scale_table", torch.zeros(4))

    model = nn.Module()
    model.blocks = nn.ModuleList([_Block()])
    counts = A.load_svdq_artifact(tmp_path / "snap", model, device="cpu", lane="dense")
    assert counts["linears"] == 3 and counts["dense"] == 3 and counts["lane"] == "dense" and counts["plain"] == 1
    assert counts["artifact"].lowrank_quant == "int8" and counts["artifact"].component == "transformer"
    dec = C.decode_int4_linear(qkv, 3 * d, d, lowrank_quant="int8")
    parts = C.split_decoded(dec, (d, d, d))
    for mod, part in zip((model.blocks[0].attn.to_q, model.blocks[0].attn.to_k, model.blocks[0].attn.to_v), parts):
        assert torch.equal(mod.weight, C.fold_decoded(part, device="cpu").weight)
    assert torch.equal(model.blocks[0].scale_table, torch.arange(4.0))
