"""Whole-checkpoint loading for the nvfp4 lane (``gen_worker_amd.nvfp4_checkpoint``), against the reference's
``load_w4a4_denoiser`` / ``swap_w4a4_linears`` / ``sanitize_w4a4_state_dict`` (``models/w4a4.py:420-664``).

Dequantization is pinned bit for bit against the oracle's independent decoder (``oracle/nvfp4_oracle.py``
``dequantize``: e2m1 table x e4m3 scale x weight_scale_2, the reference's order); the loader is checked on a
small skeleton written to a safetensors file: which layers are quantized, which run on ``Nvfp4Linear`` and
which stay dequantized (dense lane, a Linear subclass, in_features % 32), biases and plain tensors, key maps,
and refusals (shape mismatch, a checkpoint tensor with no home, a model tensor left unset). The CPU tests use
the dense lane; the GPU test swaps and compares the loaded model with the same layers built by hand.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import nvfp4_oracle as NO


class SubLinear(nn.Linear):
    """A Linear subclass: the loader must not swap it."""


class Tiny(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.lin0 = nn.Linear(64, 32)               # aligned, bias
        self.lin1 = nn.Linear(32, 48, bias=False)   # aligned, static input_scale + pre_quant_scale
        self.lin2 = nn.Linear(48, 16)               # in_features % 32 != 0: stays dequantized
        self.norm = nn.LayerNorm(16)
        self.sub = nn.Module()
        self.sub.lin3 = SubLinear(64, 16)           # not a plain Linear: stays dequantized

    def forward(self, x):
        y = self.norm(self.lin2(self.lin1(self.lin0(x))))
        return torch.cat((y, self.sub.lin3(x)), dim=-1)


QUANTIZED = ("lin0", "lin1", "lin2", "sub.lin3")


def _triple(n, k, seed):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    packed, scales, ws2 = NO.quantize_nvfp4_tensor(w)
    return packed, scales, ws2


def _checkpoint(tmp_path, prefix=""):
    """A safetensors file for ``Tiny``: every Linear quantized (flat e4m3 scales), plain norm tensors."""
    from safetensors.torch import save_file

    sd = {}
    shapes = {"lin0": (32, 64), "lin1": (48, 32), "lin2": (16, 48), "sub.lin3": (16, 64)}
    g = np.random.default_rng(3)
    for i, (name, (n, k)) in enumerate(shapes.items()):
        packed, scales, ws2 = _triple(n, k, seed=10 + i)
        sd[f"{prefix}{name}.weight"] = torch.from_numpy(packed)
        sd[f"{prefix}{name}.weight_scale"] = torch.from_numpy(scales).view(torch.float8_e4m3fn)
        sd[f"{prefix}{name}.weight_scale_2"] = torch.tensor(float(ws2), dtype=torch.float32)
        if name != "lin1":
            sd[f"{prefix}{name}.bias"] = torch.from_numpy((g.standard_normal(n) * 0.1).astype(np.float32)).to(
                torch.bfloat16)
    sd[f"{prefix}lin1.input_scale"] = torch.tensor([[0.02]], dtype=torch.float32)
    sd[f"{prefix}lin1.pre_quant_scale"] = torch.from_numpy(g.uniform(0.5, 2.0, 32).astype(np.float32)).to(
        torch.bfloat16)
    sd[f"{prefix}norm.weight"] = torch.ones(16, dtype=torch.float32) * 1.5
    sd[f"{prefix}norm.bias"] = torch.full((16,), 0.25, dtype=torch.float32)
    path = tmp_path / "denoiser.safetensors"
    save_file(sd, str(path))
    return path, sd


def _meta_skeleton():
    with torch.device("meta"):
        return Tiny()


def test_dequantize_matches_the_oracle_bit_for_bit():
    from gen_worker_amd.nvfp4 import to_blocked_scales
    from gen_worker_amd.nvfp4_checkpoint import dequantize_nvfp4_tensor

    for n, k, seed in ((32, 64, 1), (48, 160, 2), (5, 16, 3)):
        packed, scales, ws2 = _triple(n, k, seed)
        ref = NO.dequantize(packed, scales, float(ws2))
        sc = torch.from_numpy(scales).view(torch.float8_e4m3fn)
        got = dequantize_nvfp4_tensor(torch.from_numpy(packed), sc, torch.tensor(float(ws2)))
        assert got.dtype == torch.float32 and np.array_equal(got.numpy(), ref)
        got_b = dequantize_nvfp4_tensor(torch.from_numpy(packed), to_blocked_scales(sc), torch.tensor(float(ws2)))
        assert np.array_equal(got_b.numpy(), ref)   # the blocked scale layout decodes the same


def test_scan_and_sanitize(tmp_path):
    from gen_worker_amd.nvfp4_checkpoint import sanitize_nvfp4_state_dict, scan_nvfp4_artifact

    path, sd = _checkpoint(tmp_path)
    art = scan_nvfp4_artifact([path])
    assert art.quantized == tuple(sorted(QUANTIZED))
    assert art.static_input_scales and art.pre_quant_scales
    clean = sanitize_nvfp4_state_dict(sd, torch.bfloat16)
    assert not any(k.endswith(("weight_scale", "weight_scale_2", "input_scale", "pre_quant_scale")) for k in clean)
    assert set(clean) == {k for k in sd if not k.endswith(("weight_scale", "weight_scale_2", "input_scale",
                                                           "pre_quant_scale"))}
    # lin1: code * scale * ws2 in fp32, times pre_quant_scale along the inputs, then bf16
    ref = NO.dequantize(sd["lin1.weight"].numpy(), sd["lin1.weight_scale"].view(torch.uint8).numpy(),
                        float(sd["lin1.weight_scale_2"])) * sd["lin1.pre_quant_scale"].float().numpy()[None, :]
    assert clean["lin1.weight"].dtype == torch.bfloat16
    assert torch.equal(clean["lin1.weight"], torch.from_numpy(ref.astype(np.float32)).to(torch.bfloat16))
    assert torch.equal(clean["norm.weight"], sd["norm.weight"])   # plain tensors pass through


def test_load_dense_lane_equals_the_sanitized_state_dict(tmp_path):
    from gen_worker_amd.nvfp4_checkpoint import load_nvfp4_denoiser, sanitize_nvfp4_state_dict

    path, sd = _checkpoint(tmp_path)
    model = _meta_skeleton()
    counts = load_nvfp4_denoiser([path], model, device="cpu", lane="dense")
    assert counts["swapped"] == 0 and counts["dequantized"] == {"dense_lane": 4} and counts["plain"] == 2
    ref = Tiny().to(torch.bfloat16)
    ref.load_state_dict({k: v.to(torch.bfloat16) for k, v in sanitize_nvfp4_state_dict(sd).items()})
    x = torch.randn(5, 64).to(torch.bfloat16)
    with torch.no_grad():
        assert torch.equal(model(x), ref(x))
    assert all(not p.is_meta for p in model.parameters())


def test_key_map_and_refusals(tmp_path):
    from gen_worker_amd.nvfp4_checkpoint import Nvfp4CheckpointError, load_nvfp4_denoiser

    path, sd = _checkpoint(tmp_path, prefix="transformer.")
    strip = lambda name: name[len("transformer."):] if name.startswith("transformer.") else name  # noqa: E731
    counts = load_nvfp4_denoiser([path], _meta_skeleton(), key_map=strip, device="cpu", lane="dense")
    assert counts["plain"] == 2
    with pytest.raises(Nvfp4CheckpointError, match="no module"):
        load_nvfp4_denoiser([path], _meta_skeleton(), device="cpu", lane="dense")   # names do not resolve
    bad = _meta_skeleton()
    bad.lin0 = nn.Linear(64, 48, device="meta")
    with pytest.raises(Nvfp4CheckpointError, match="is \\[32, 64\\] in the checkpoint"):
        load_nvfp4_denoiser([path], bad, key_map=strip, device="cpu", lane="dense")
    extra = _meta_skeleton()
    extra.register_buffer("unset", torch.empty(3, device="meta"))
    with pytest.raises(Nvfp4CheckpointError, match="unset"):
        load_nvfp4_denoiser([path], extra, key_map=strip, device="cpu", lane="dense")
    small = _meta_skeleton()
    del small.norm
    small.norm = nn.Identity()
    with pytest.raises(Nvfp4CheckpointError, match="no parameter or buffer"):
        load_nvfp4_denoiser([path], small, key_map=strip, device="cpu", lane="dense")
    with pytest.raises(ValueError, match="lane"):
        load_nvfp4_denoiser([path], _meta_skeleton(), key_map=strip, device="cpu", lane="fp4")
    # bias presence must agree (the reference's load_state_dict reports either side's extra bias), in the
    # swap branch (lane nvfp4: refused before any module is built) and the dequantized one
    from safetensors.torch import save_file

    no_b0 = tmp_path / "no_lin0_bias.safetensors"
    save_file({k: v for k, v in sd.items() if k != "transformer.lin0.bias"}, str(no_b0))
    for lane in ("nvfp4", "dense"):   # lin0 is the first layer swapped: nothing is built before the check
        nobias = _meta_skeleton()
        nobias.lin0 = nn.Linear(64, 32, bias=False, device="meta")     # the checkpoint has lin0.bias
        with pytest.raises(Nvfp4CheckpointError, match="no bias"):
            load_nvfp4_denoiser([path], nobias, key_map=strip, device="cpu", lane=lane)
        with pytest.raises(Nvfp4CheckpointError, match="does not provide"):   # module bias, none stored
            load_nvfp4_denoiser([no_b0], _meta_skeleton(), key_map=strip, device="cpu", lane=lane)


@pytest.mark.gpu
def test_load_nvfp4_lane_swaps_what_can_run_quantized(tmp_path):
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native
    from gen_worker_amd.nvfp4 import Nvfp4Linear, build_nvfp4_linear
    from gen_worker_amd.nvfp4_checkpoint import dequantize_nvfp4_tensor, load_nvfp4_denoiser

    _native.load()
    path, sd = _checkpoint(tmp_path)
    model = _meta_skeleton()
    counts = load_nvfp4_denoiser([path], model, device="cuda", lane="nvfp4")
    assert counts["swapped"] == 2
    assert counts["dequantized"] == {"dim_unaligned": 1, "not_plain_linear": 1}
    assert isinstance(model.lin0, Nvfp4Linear) and isinstance(model.lin1, Nvfp4Linear)
    assert type(model.lin2) is nn.Linear and type(model.sub.lin3) is SubLinear
    assert model.lin1.input_scale is not None and model.lin1.pre_quant_scale is not None

    # the same model assembled by hand from the contract tensors
    ref = Tiny().to("cuda", torch.bfloat16)
    for name in ("lin0", "lin1"):
        setattr(ref, name, build_nvfp4_linear(sd[f"{name}.weight"], sd[f"{name}.weight_scale"],
                                              sd[f"{name}.weight_scale_2"], bias=sd.get(f"{name}.bias"),
                                              input_scale=sd.get(f"{name}.input_scale"),
                                              pre_quant_scale=sd.get(f"{name}.pre_quant_scale"), device="cuda"))
    with torch.no_grad():
        for mod, name in ((ref.lin2, "lin2"), (ref.sub.lin3, "sub.lin3")):
            mod.weight.copy_(dequantize_nvfp4_tensor(sd[f"{name}.weight"], sd[f"{name}.weight_scale"],
                                                     sd[f"{name}.weight_scale_2"]).to(torch.bfloat16))
            mod.bias.copy_(sd[f"{name}.bias"])
        ref.norm.weight.copy_(sd["norm.weight"])
        ref.norm.bias.copy_(sd["norm.bias"])
        x = torch.randn(40, 64, device="cuda").to(torch.bfloat16)
        y, y_ref = model(x), ref(x)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
