"""W8A8 lane qualification and whole-checkpoint loading (``gen_worker_amd.qualify`` W8A8 gate,
``gen_worker_amd.w8a8.serving_w8a8_linear``, ``gen_worker_amd.w8a8_checkpoint``), against the reference's
``w8a8_gemm_mode`` / ``load_w8a8_denoiser`` / ``swap_w8a8_linears`` / ``sanitize_w8a8_state_dict`` /
``quantize_tree_w8a8`` (``models/w8a8.py:137-792``).

The gate's decision rule runs with its probe and timing stubbed (no GPU here): branch order, the 1.10x bar,
a failing probe or a raising bench moving to the next branch, and the dequant lane when none qualifies. The
loader is checked on a small skeleton written to safetensors files: which layers are quantized (int8 and
e4m3 weights with a ``weight_scale`` twin), which run on ``Int8ScaledLinear`` and which are served
dequantized (the dequant lane, e4m3 weights, a Linear subclass, in_features % 64), biases, plain tensors,
key maps and refusals. Codes and scales the producer writes are pinned byte for byte against the oracle's
int8 weight quantizer; dequantization against the oracle's codes x scales in float32.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import svdq_oracle as O


class SubLinear(nn.Linear):
    """A Linear subclass: the loader must not swap it."""


class Tiny(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.lin0 = nn.Linear(128, 64)              # aligned, bias
        self.lin1 = nn.Linear(64, 32, bias=False)   # aligned, static input_scale
        self.lin2 = nn.Linear(32, 16)               # in_features % 64 != 0: dequantized
        self.lin3 = nn.Linear(64, 16)               # e4m3 weights: dequantized
        self.norm = nn.LayerNorm(16)
        self.sub = nn.Module()
        self.sub.lin4 = SubLinear(128, 16)          # not a plain Linear: dequantized


SHAPES = {"lin0": (64, 128), "lin1": (32, 64), "lin2": (16, 32), "lin3": (16, 64), "sub.lin4": (16, 128)}


def _checkpoint(tmp_path, prefix="", name="denoiser.safetensors"):
    from safetensors.torch import save_file

    g = np.random.default_rng(5)
    sd = {}
    for i, (layer, (n, k)) in enumerate(SHAPES.items()):
        w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
        q, s = O.quantize_weight_int8(w)
        if layer == "lin3":   # the reference's own format: e4m3 codes, per-channel scale
            t = torch.from_numpy(w / s).clamp(-448, 448).to(torch.float8_e4m3fn)
        else:
            t = torch.from_numpy(q)
        sd[f"{prefix}{layer}.weight"] = t
        sd[f"{prefix}{layer}.weight_scale"] = torch.from_numpy(s.reshape(-1) if i % 2 else s)  # [n] or [n, 1]
        if layer != "lin1":
            sd[f"{prefix}{layer}.bias"] = torch.from_numpy((g.standard_normal(n) * 0.1).astype(np.float32))
    sd[f"{prefix}lin1.input_scale"] = torch.tensor([[0.02]], dtype=torch.float32)
    sd[f"{prefix}norm.weight"] = torch.ones(16) * 1.5
    sd[f"{prefix}norm.bias"] = torch.full((16,), 0.25)
    path = tmp_path / name
    save_file(sd, str(path))
    return path, sd


def _meta_skeleton():
    with torch.device("meta"):
        return Tiny()


# ---------------------------------------------------------------------------
# the gate
# ---------------------------------------------------------------------------

def _stub_gate(monkeypatch, probe, speed):
    from gen_worker_amd import qualify

    monkeypatch.setattr(qualify, "extension_available", lambda: True)
    monkeypatch.setattr(qualify, "w8a8_probe", probe)
    monkeypatch.setattr(qualify, "w8a8_gemm_speedup", speed)
    return qualify


def test_w8a8_gate_takes_the_first_branch_that_qualifies(monkeypatch):
    q = _stub_gate(monkeypatch, lambda mode: None,
                   lambda mode, protocol="graph": (1.0, 1.2, 1.2) if mode == "rowwise" else (1.0, 2.0, 2.0))
    r = q.qualify_w8a8()
    assert r.mode == "rowwise" and not r.reasons
    assert set(r.timings) == {"rowwise"} and set(r.timings["rowwise"]) == {"graph", "eager"}


def test_w8a8_gate_falls_through_to_pertensor_then_dequant(monkeypatch):
    q = _stub_gate(monkeypatch, lambda mode: None,
                   lambda mode, protocol="graph": (1.0, 1.05, 1.05) if mode == "rowwise" else (1.0, 1.15, 1.15))
    r = q.qualify_w8a8()
    assert r.mode == "pertensor" and len(r.reasons) == 1 and "1.05x" in r.reasons[0]
    q = _stub_gate(monkeypatch, lambda mode: None, lambda mode, protocol="graph": (1.0, 1.09, 1.09))
    r = q.qualify_w8a8()
    assert r.mode == "" and len(r.reasons) == 2


def test_w8a8_gate_probe_failure_and_bench_error_move_on(monkeypatch):
    def bench(mode, protocol="graph"):
        if mode == "pertensor":
            raise RuntimeError("bench broke")
        return (1.0, 3.0, 3.0)

    q = _stub_gate(monkeypatch, lambda mode: "numerics off" if mode == "rowwise" else None, bench)
    r = q.qualify_w8a8()
    assert r.mode == "" and r.reasons[0] == "numerics off" and "bench broke" in r.reasons[1]


def test_w8a8_mode_resolution(monkeypatch):
    from gen_worker_amd import qualify

    assert qualify.resolve_w8a8_mode("pertensor") == "pertensor"
    assert qualify.resolve_w8a8_mode("dequant") == "dequant"
    with pytest.raises(ValueError):
        qualify.resolve_w8a8_mode("blockwise")
    monkeypatch.setattr(qualify, "w8a8_gemm_mode", lambda: "")
    assert qualify.resolve_w8a8_mode() == "dequant"
    monkeypatch.setattr(qualify, "w8a8_gemm_mode", lambda: "rowwise")
    assert qualify.resolve_w8a8_mode() == "rowwise"


def test_w8a8_gate_without_gpu_is_the_dequant_lane():
    from gen_worker_amd import qualify

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = qualify.qualify_w8a8()
    assert r.mode == "" and r.reasons


def test_w4a4_qualification_records_both_timing_protocols(monkeypatch):
    from gen_worker_amd import qualify

    monkeypatch.setattr(qualify, "extension_available", lambda: True)
    for gate in ("quantizer_bit_identical", "fused_self_check", "gemm_numerics_ok"):
        monkeypatch.setattr(qualify, gate, lambda: None)
    monkeypatch.setattr(qualify, "gemm_speedup",
                        lambda protocol="graph": (0.08, 0.1, 1.25) if protocol == "graph" else (0.1, 0.105, 1.05))
    r = qualify.qualify()
    # the decision follows the graph protocol; the reference's single-call ratio is kept beside it
    assert r.lane == "int4" and r.speedup == 1.25 and r.speedup_eager == 1.05 and r.int4_ms_eager == 0.1


# ---------------------------------------------------------------------------
# serving helper
# ---------------------------------------------------------------------------

def test_serving_linear_per_mode():
    from gen_worker_amd.w8a8 import Int8ScaledLinear, serving_w8a8_linear

    g = np.random.default_rng(1)
    w = (g.standard_normal((32, 64)) * 0.05).astype(np.float32)
    q, s = O.quantize_weight_int8(w)
    b = torch.from_numpy(g.standard_normal(32).astype(np.float32)).to(torch.bfloat16)
    lin = serving_w8a8_linear(qweight=torch.from_numpy(q), weight_scale=torch.from_numpy(s), bias=b,
                              device="cpu", mode="dequant")
    assert type(lin) is nn.Linear and lin.weight.dtype == torch.bfloat16
    want = torch.from_numpy((q.astype(np.float32) * s).astype(np.float32)).to(torch.bfloat16)
    assert torch.equal(lin.weight, want) and torch.equal(lin.bias, b)
    mod = serving_w8a8_linear(qweight=torch.from_numpy(q), weight_scale=torch.from_numpy(s), bias=b, device="cpu",
                              mode="pertensor")
    assert isinstance(mod, Int8ScaledLinear) and mod.gemm_mode == "pertensor"
    assert np.array_equal(mod.weight.numpy(), q) and np.array_equal(mod.weight_scale.numpy(), s)


# ---------------------------------------------------------------------------
# the loader
# ---------------------------------------------------------------------------

def test_scan_detects_int8_and_fp8_layers(tmp_path):
    from gen_worker_amd.w8a8_checkpoint import scan_w8a8_artifact

    path, _ = _checkpoint(tmp_path)
    art = scan_w8a8_artifact([path])
    assert art.quantized == tuple(sorted(SHAPES)) and art.fp8 == ("lin3",) and art.static_input_scales


def test_dequantize_and_sanitize_match_the_oracle(tmp_path):
    from gen_worker_amd.w8a8_checkpoint import dequantize_w8a8_tensor, sanitize_w8a8_state_dict

    _, sd = _checkpoint(tmp_path)
    out = sanitize_w8a8_state_dict(sd, torch.float32)
    assert not any(k.endswith((".weight_scale", ".input_scale")) for k in out)
    for layer in SHAPES:
        w, s = sd[f"{layer}.weight"], sd[f"{layer}.weight_scale"]
        want = w.float().numpy() * s.numpy().reshape(-1, 1)
        assert np.array_equal(out[f"{layer}.weight"].numpy(), want), layer
        assert np.array_equal(dequantize_w8a8_tensor(w, s).numpy(), want)
    assert torch.equal(out["norm.weight"], sd["norm.weight"])


def test_load_dequant_lane_equals_the_sanitized_state_dict(tmp_path):
    from gen_worker_amd.w8a8_checkpoint import load_w8a8_denoiser, sanitize_w8a8_state_dict

    path, sd = _checkpoint(tmp_path)
    model = _meta_skeleton()
    counts = load_w8a8_denoiser([path], model, device="cpu", mode="dequant", compute_dtype=torch.float32)
    assert counts["swapped"] == 0 and counts["dequantized"] == {"dequant_lane": len(SHAPES)}
    assert counts["plain"] == 2 and counts["mode"] == "dequant"
    ref = sanitize_w8a8_state_dict(sd, torch.float32)
    got = model.state_dict()
    for k, v in ref.items():
        assert torch.equal(got[k], v), k


def test_load_w8a8_lane_swaps_what_can_run_quantized(tmp_path):
    from gen_worker_amd.w8a8 import Int8ScaledLinear
    from gen_worker_amd.w8a8_checkpoint import load_w8a8_denoiser

    path, sd = _checkpoint(tmp_path)
    model = _meta_skeleton()
    counts = load_w8a8_denoiser([path], model, device="cpu", mode="rowwise")
    assert counts["swapped"] == 2
    assert counts["dequantized"] == {"dim_unaligned": 1, "fp8_weight": 1, "not_plain_linear": 1}
    for layer in ("lin0", "lin1"):
        mod = model.get_submodule(layer)
        assert isinstance(mod, Int8ScaledLinear) and mod.gemm_mode == "rowwise"
        assert torch.equal(mod.weight, sd[f"{layer}.weight"])
        assert torch.equal(mod.weight_scale.reshape(-1), sd[f"{layer}.weight_scale"].reshape(-1))
    assert model.lin1.input_scale.item() == pytest.approx(0.02) and model.lin1.bias is None
    assert torch.equal(model.lin0.bias, sd["lin0.bias"].to(torch.bfloat16))
    assert type(model.lin2) is nn.Linear and model.lin2.weight.dtype == torch.bfloat16
    assert isinstance(model.sub.lin4, SubLinear)


def test_key_map_and_refusals(tmp_path):
    from gen_worker_amd.w8a8_checkpoint import (W8a8CheckpointError, load_w8a8_denoiser, scan_w8a8_artifact,
                                                swap_w8a8_linears)

    path, _ = _checkpoint(tmp_path, prefix="transformer.")
    model = _meta_skeleton()
    strip = lambda name: name[len("transformer."):]  # noqa: E731
    counts = load_w8a8_denoiser([path], model, device="cpu", mode="dequant", key_map=strip)
    assert counts["plain"] == 2 and not any(p.is_meta for p in model.parameters())
    # a checkpoint bias on a module without one
    path2, _ = _checkpoint(tmp_path, name="b.safetensors")
    built = Tiny()
    built.lin0 = nn.Linear(128, 64, bias=False)
    with pytest.raises(W8a8CheckpointError, match="no bias"):
        swap_w8a8_linears(built, scan_w8a8_artifact([path2]), device="cpu", mode="dequant")
    # a module bias on meta that the checkpoint does not provide
    model = _meta_skeleton()
    with torch.device("meta"):
        model.lin1 = nn.Linear(64, 32, bias=True)
    with pytest.raises(W8a8CheckpointError, match="does not provide"):
        swap_w8a8_linears(model, scan_w8a8_artifact([path2]), device="cpu", mode="rowwise")
    # shape mismatch
    model = _meta_skeleton()
    with torch.device("meta"):
        model.lin0 = nn.Linear(128, 48)
    with pytest.raises(W8a8CheckpointError, match="checkpoint"):
        swap_w8a8_linears(model, scan_w8a8_artifact([path2]), device="cpu", mode="dequant")
    with pytest.raises(W8a8CheckpointError, match="no W8A8 layer"):
        from safetensors.torch import save_file

        save_file({"a.weight": torch.ones(4, 4)}, str(tmp_path / "plain.safetensors"))
        scan_w8a8_artifact([tmp_path / "plain.safetensors"])


def test_producer_tree_round_trip_matches_the_oracle(tmp_path):
    from safetensors.torch import load_file, save_file

    from gen_worker_amd.w8a8_checkpoint import detect_w8a8_artifacts, quantize_tree_w8a8

    src = tmp_path / "src"
    (src / "transformer").mkdir(parents=True)
    (src / "vae").mkdir()
    (src / "model_index.json").write_text(json.dumps({"transformer": ["diffusers", "X"]}))
    (src / "transformer" / "config.json").write_text("{}")
    g = np.random.default_rng(9)
    blocks = {"blocks.0.attn.to_q.weight": (g.standard_normal((64, 128)) * 0.02).astype(np.float32),
              "blocks.0.norm.weight": np.ones((64, 64), np.float32),        # excluded by name
              "pos_embed.proj.weight": (g.standard_normal((32, 64))).astype(np.float32),  # excluded
              "blocks.0.ff.weight": (g.standard_normal((48, 40))).astype(np.float32),  # 40 % 16 != 0
              "blocks.0.attn.to_q.bias": g.standard_normal(64).astype(np.float32)}
    save_file({k: torch.from_numpy(v) for k, v in blocks.items()}, str(src / "transformer" / "m.safetensors"))
    save_file({"dec.weight": torch.ones(16, 16)}, str(src / "vae" / "v.safetensors"))
    out = quantize_tree_w8a8(src, tmp_path / "out")
    arts = detect_w8a8_artifacts(out)
    assert [c for c, _ in arts] == ["transformer"] and arts[0][1].quantized == ("blocks.0.attn.to_q",)
    t = load_file(str(out / "transformer" / "m.safetensors"))
    q, s = O.quantize_weight_int8(blocks["blocks.0.attn.to_q.weight"])
    assert np.array_equal(t["blocks.0.attn.to_q.weight"].numpy(), q)
    assert np.array_equal(t["blocks.0.attn.to_q.weight_scale"].numpy(), s.reshape(-1))
    assert t["blocks.0.norm.weight"].dtype == torch.float32 and t["blocks.0.ff.weight"].dtype == torch.float32
    assert json.loads((out / "transformer" / "config.json").read_text())["quantization_config"]["quant_algo"] == "INT8"
    assert torch.equal(load_file(str(out / "vae" / "v.safetensors"))["dec.weight"], torch.ones(16, 16))
