"""Whole-denoiser loading for the nvfp4 compatibility lane.

The reference serves modelopt nvfp4 checkpoints (its ``cozy.nvfp4-flat@1`` rule) three ways
(``src/gen_worker/models/w4a4.py``): materialize a denoiser skeleton and assign the shards' tensors,
swapping each quantized ``nn.Linear`` for its W4A4 module or dequantizing it where it cannot run quantized
(``load_w4a4_denoiser``, ``:420-498``); swap the quantized Linears of an already-built model
(``swap_w4a4_linears``, ``:559-664``); and dequantize a raw state dict for loaders that build the model
themselves (``sanitize_w4a4_state_dict``, ``:523-556``). A quantized layer ``L`` is the triple
``L.weight`` (uint8 [out, in/2], e2m1 codes, element 2j in the low nibble), ``L.weight_scale`` (e4m3
[out, in/16], flat row-major) and ``L.weight_scale_2`` (fp32 scalar), with optional ``L.input_scale``
(static activation second-level scale) and ``L.pre_quant_scale`` ([in], multiplies the activations).

Here the quantized module is ``Nvfp4Linear`` (``nvfp4.py``: the reference's activation codes, products on
exact bf16 values). A layer stays dequantized (code * scale * weight_scale_2 in fp32, times
``pre_quant_scale`` along the inputs, cast to the compute dtype) when the module in its place is not a
plain ``nn.Linear``, when in_features % 32 or out_features % 16 (the reference's alignment), or when the
caller asks for the dense lane. Tensors are read with safetensors only (nothing is unpickled).
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Callable, Dict, Iterable, Optional, Sequence

import torch
import torch.nn as nn
from torch import Tensor

from .nvfp4 import BLOCK, build_nvfp4_linear, from_blocked_scales

logger = logging.getLogger(__name__)

AUX_SUFFIXES = (".weight_scale", ".weight_scale_2", ".input_scale", ".pre_quant_scale")
K_ALIGN, N_ALIGN = 32, 16  # models/w4a4.py _K_ALIGN / _N_ALIGN
LANES = ("nvfp4", "dense")
_E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


class Nvfp4CheckpointError(ValueError):
    """The checkpoint does not match the nvfp4 contract or the model it is loaded into."""


@dataclass(frozen=True)
class Nvfp4Artifact:
    """The shards of an nvfp4 checkpoint and what they hold (the reference's ``W4a4Artifact`` fields this
    lane uses)."""

    files: tuple[Path, ...]
    quantized: tuple[str, ...]
    static_input_scales: bool
    pre_quant_scales: bool


def quantized_layers(names: Iterable[str], dtype_of: Callable[[str], str]) -> tuple[str, ...]:
    """Layer names carrying a complete nvfp4 triple: ``L.weight_scale_2`` present, ``L.weight_scale`` present
    and ``L.weight`` of dtype uint8 (``dtype_of`` returns a safetensors dtype string or a torch dtype name)."""
    names = set(names)
    out = []
    for key in names:
        if not key.endswith(".weight_scale_2"):
            continue
        layer = key[: -len(".weight_scale_2")]
        if f"{layer}.weight" in names and f"{layer}.weight_scale" in names and \
                str(dtype_of(f"{layer}.weight")).lower() in ("u8", "uint8", "torch.uint8"):
            out.append(layer)
    return tuple(sorted(out))


def scan_nvfp4_artifact(files: Sequence[Any]) -> Nvfp4Artifact:
    """Read the shards' headers (no tensor data) and list the quantized layers."""
    from safetensors import safe_open

    paths = tuple(Path(f) for f in files)
    dtypes: Dict[str, str] = {}
    for p in paths:
        with safe_open(str(p), framework="pt", device="cpu") as fh:
            for name in fh.keys():
                if name in dtypes:
                    raise Nvfp4CheckpointError(f"tensor {name!r} appears in more than one shard")
                dtypes[name] = fh.get_slice(name).get_dtype()
    quantized = quantized_layers(dtypes, dtypes.__getitem__)
    if not quantized:
        raise Nvfp4CheckpointError(f"no nvfp4 layer (uint8 weight + weight_scale + weight_scale_2) in {len(paths)} shard(s)")
    return Nvfp4Artifact(paths, quantized, any(f"{q}.input_scale" in dtypes for q in quantized),
                         any(f"{q}.pre_quant_scale" in dtypes for q in quantized))


def _e2m1_values(packed: Tensor) -> Tensor:
    """uint8 [n, k/2] -> float32 [n, k]: element 2j from the low nibble of byte j (bit 3 the sign)."""
    lut = torch.tensor(_E2M1 + tuple(-v for v in _E2M1), dtype=torch.float32, device=packed.device)
    p = packed.to(torch.int64)
    return torch.stack((lut[p & 0xF], lut[p >> 4]), dim=-1).reshape(packed.shape[0], -1)


def dequantize_nvfp4_tensor(weight: Tensor, weight_scale: Tensor, weight_scale_2: Tensor) -> Tensor:
    """The contract triple -> float32 [out, in] = code * scale * weight_scale_2 (the reference's order,
    ``models/w4a4.py:157-164``: code * scale is exact in fp32, the second factor rounds once).
    ``weight_scale`` flat [out, in/16] or in the blocked layout."""
    if weight.dtype != torch.uint8 or weight.dim() != 2:
        raise Nvfp4CheckpointError(f"weight must be uint8 [out, in/2], got {weight.dtype} {tuple(weight.shape)}")
    n, k = int(weight.shape[0]), 2 * int(weight.shape[1])
    if k % BLOCK:
        raise Nvfp4CheckpointError(f"in_features {k} is not a multiple of {BLOCK}")
    kb = k // BLOCK
    sc = weight_scale if weight_scale.dtype == torch.float8_e4m3fn else weight_scale.view(torch.float8_e4m3fn)
    if sc.numel() != n * kb or (sc.dim() == 2 and tuple(sc.shape) != (n, kb)):
        sc = from_blocked_scales(sc, n, kb)
    vals = _e2m1_values(weight).reshape(n, kb, BLOCK)
    return (vals * sc.float().reshape(n, kb, 1) * weight_scale_2.float().reshape(())).reshape(n, k)


def _dense_weight(tensors: Dict[str, Tensor], layer: str, dtype: torch.dtype) -> Tensor:
    w = dequantize_nvfp4_tensor(tensors[f"{layer}.weight"], tensors[f"{layer}.weight_scale"],
                                tensors[f"{layer}.weight_scale_2"])
    pqs = tensors.get(f"{layer}.pre_quant_scale")
    if pqs is not None:
        w = w * pqs.float().reshape(1, -1)
    return w.to(dtype)


def sanitize_nvfp4_state_dict(state_dict: Dict[str, Tensor], compute_dtype: torch.dtype = torch.bfloat16
                              ) -> Dict[str, Tensor]:
    """A raw state dict with every nvfp4 triple dequantized into ``L.weight`` of ``compute_dtype`` (the
    pre-quant scale folded in) and the quantized layers' auxiliary tensors dropped; other tensors as given
    (``sanitize_w4a4_state_dict``, ``models/w4a4.py:523-556``)."""
    quantized = set(quantized_layers(state_dict, lambda k: state_dict[k].dtype))
    out: Dict[str, Tensor] = {}
    for key, t in state_dict.items():
        if key.endswith(".weight") and key[: -len(".weight")] in quantized:
            out[key] = _dense_weight(state_dict, key[: -len(".weight")], compute_dtype)
        elif any(key.endswith(s) and key[: -len(s)] in quantized for s in AUX_SUFFIXES):
            continue
        else:
            out[key] = t
    return out


def _module_at(model: nn.Module, path: str) -> tuple[nn.Module, str, Any]:
    parent_path, _, leaf = path.rpartition(".")
    try:
        parent = model.get_submodule(parent_path) if parent_path else model
        return parent, leaf, getattr(parent, leaf)
    except AttributeError as exc:
        raise Nvfp4CheckpointError(f"no module {path!r} in {type(model).__name__}") from exc


def _swap_reason(old: Any, out_f: int, in_f: int, lane: str) -> Optional[str]:
    """Why a layer stays dequantized (None: it runs on Nvfp4Linear)."""
    if lane == "dense":
        return "dense_lane"
    if type(old) is not nn.Linear:
        return "not_plain_linear"
    if in_f % K_ALIGN or out_f % N_ALIGN:
        return "dim_unaligned"
    return None


class _ShardReader:
    """Tensors by name across the artifact's shards, each file opened once."""

    def __init__(self, files: Sequence[Path]) -> None:
        from safetensors import safe_open

        self._handles = [safe_open(str(f), framework="pt", device="cpu") for f in files]
        self.where: Dict[str, Any] = {}
        for fh in self._handles:
            for name in fh.keys():
                self.where[name] = fh

    def get(self, name: str) -> Tensor:
        fh = self.where.get(name)
        if fh is None:
            raise Nvfp4CheckpointError(f"artifact tensor {name!r} missing from the shards")
        return fh.get_tensor(name)

    def layer(self, layer: str) -> Dict[str, Tensor]:
        return {f"{layer}{s}": self.get(f"{layer}{s}") for s in (".weight", ".bias") + AUX_SUFFIXES
                if f"{layer}{s}" in self.where}


def _layer_bias(layer: str, target: str, tensors: Dict[str, Tensor], old: Any) -> Optional[Tensor]:
    """The layer's bias: the checkpoint's ``L.bias`` when the module has a bias, else the module's own when it
    is materialized. A checkpoint bias on a module without one, or a module bias that neither provides, raises
    (the reference builds the module with ``bias=old.bias is not None`` and its ``load_state_dict`` reports
    both as unexpected / missing keys, ``models/w4a4.py:488-493``)."""
    ckpt = tensors.get(f"{layer}.bias")
    mod_bias = getattr(old, "bias", None)
    if mod_bias is None:
        if ckpt is not None:
            raise Nvfp4CheckpointError(f"checkpoint has {layer}.bias but module {target!r} has no bias")
        return None
    if ckpt is not None:
        return ckpt
    if mod_bias.is_meta:
        raise Nvfp4CheckpointError(f"module {target!r} has a bias the checkpoint does not provide")
    return mod_bias.detach()


def _check_lane(lane: str) -> str:
    if lane not in LANES:
        raise ValueError(f"lane {lane!r} is not one of {LANES}")
    return lane


def swap_nvfp4_linears(model: nn.Module, art: Nvfp4Artifact, *, key_map: Optional[Callable[[str], str]] = None,
                       device: Any = "cuda", lane: str = "nvfp4",
                       compute_dtype: torch.dtype = torch.bfloat16) -> dict:
    """Swap the artifact's quantized layers in an already-built ``model`` (``swap_w4a4_linears``): each plain,
    aligned ``nn.Linear`` becomes an ``Nvfp4Linear``; any other keeps its module with the dequantized weight
    assigned. The bias is the checkpoint's ``L.bias`` when it has one, else the module's (``_layer_bias``: a
    bias only one side has raises). ``key_map`` maps an
    artifact layer name to the model's module path. Returns {"quantized", "swapped", "dequantized":
    {reason: count}}; a shape mismatch raises."""
    _check_lane(lane)
    reader = _ShardReader(art.files)
    counts: Dict[str, Any] = {"quantized": len(art.quantized), "swapped": 0, "dequantized": {}}
    for layer in art.quantized:
        target = key_map(layer) if key_map is not None else layer
        parent, leaf, old = _module_at(model, target)
        tensors = reader.layer(layer)
        w = tensors[f"{layer}.weight"]
        out_f, in_f = int(w.shape[0]), 2 * int(w.shape[1])
        mod_shape = (getattr(old, "out_features", None), getattr(old, "in_features", None))
        if mod_shape != (out_f, in_f):
            raise Nvfp4CheckpointError(f"layer {layer!r} is [{out_f}, {in_f}] in the checkpoint, module {target!r} "
                                       f"is {list(mod_shape)}")
        why = _swap_reason(old, out_f, in_f, lane)
        bias = _layer_bias(layer, target, tensors, old)
        if why is None:
            new = build_nvfp4_linear(w, tensors[f"{layer}.weight_scale"], tensors[f"{layer}.weight_scale_2"],
                                     bias=bias, input_scale=tensors.get(f"{layer}.input_scale"),
                                     pre_quant_scale=tensors.get(f"{layer}.pre_quant_scale"), device=device)
            setattr(parent, leaf, new)
            counts["swapped"] += 1
        else:
            dense = _dense_weight(tensors, layer, compute_dtype).to(device)
            old.weight = nn.Parameter(dense, requires_grad=False)
            if bias is not None:
                old.bias = nn.Parameter(bias.to(device=device, dtype=compute_dtype), requires_grad=False)
            counts["dequantized"][why] = counts["dequantized"].get(why, 0) + 1
    partial = {k: v for k, v in counts["dequantized"].items() if k != "dense_lane"}
    if partial:
        logger.warning("nvfp4 swap: %d/%d quantized layers on Nvfp4Linear, %s stayed dequantized",
                       counts["swapped"], counts["quantized"],
                       ", ".join(f"{k}={v}" for k, v in sorted(partial.items())))
    return counts


def load_nvfp4_denoiser(art: Any, model: nn.Module, *, key_map: Optional[Callable[[str], str]] = None,
                        device: Any = "cuda", lane: str = "nvfp4",
                        compute_dtype: torch.dtype = torch.bfloat16) -> dict:
    """Materialize ``model`` (a skeleton whose parameters may sit on the meta device) from an nvfp4
    checkpoint (``load_w4a4_denoiser``): the quantized layers through ``swap_nvfp4_linears``, every other
    tensor assigned to the parameter or buffer of its name (floating tensors in ``compute_dtype``, fp8 kept).
    A checkpoint tensor with no home, a shape mismatch, or a model tensor the checkpoint leaves unset raises.
    ``art``: an ``Nvfp4Artifact`` or the shard paths. Returns the swap counts plus {"plain": n}."""
    if not isinstance(art, Nvfp4Artifact):
        art = scan_nvfp4_artifact(art if isinstance(art, (list, tuple)) else [art])
    counts = swap_nvfp4_linears(model, art, key_map=key_map, device=device, lane=lane, compute_dtype=compute_dtype)
    claimed = set()
    for layer in art.quantized:
        claimed.update(f"{layer}{s}" for s in (".weight", ".bias") + AUX_SUFFIXES)
    reader = _ShardReader(art.files)
    mapped: Dict[str, str] = {}
    for name in reader.where:
        if name in claimed:
            continue
        prefix, _, leaf = name.rpartition(".")
        if key_map is not None:
            target = f"{key_map(prefix)}.{leaf}" if prefix else name
        else:
            target = name
        mapped[name] = target
    homes = dict(model.named_parameters())
    homes.update(dict(model.named_buffers()))
    plain = 0
    with torch.no_grad():
        for name, target in mapped.items():
            if target not in homes:
                raise Nvfp4CheckpointError(f"checkpoint tensor {name!r} has no parameter or buffer {target!r} in "
                                           f"{type(model).__name__}")
            t = reader.get(name)
            dst = homes[target]
            if tuple(dst.shape) != tuple(t.shape):
                raise Nvfp4CheckpointError(f"{name!r}: checkpoint shape {tuple(t.shape)} != model {tuple(dst.shape)}")
            if t.is_floating_point() and t.dtype != torch.float8_e4m3fn:
                t = t.to(compute_dtype)
            owner_path, _, leaf = target.rpartition(".")
            owner = model.get_submodule(owner_path) if owner_path else model
            new = t.to(device)
            if isinstance(dst, nn.Parameter):
                setattr(owner, leaf, nn.Parameter(new, requires_grad=False))
            else:
                owner.register_buffer(leaf, new)
            plain += 1
    missing = [n for n, p in list(model.named_parameters()) + list(model.named_buffers()) if p.is_meta]
    if missing:
        raise Nvfp4CheckpointError(f"the checkpoint leaves {len(missing)} model tensor(s) unset, e.g. {missing[:5]}")
    model.eval()
    counts["plain"] = plain
    return counts


__all__ = ["AUX_SUFFIXES", "K_ALIGN", "LANES", "N_ALIGN", "Nvfp4Artifact", "Nvfp4CheckpointError",
           "dequantize_nvfp4_tensor", "load_nvfp4_denoiser", "quantized_layers", "sanitize_nvfp4_state_dict",
           "scan_nvfp4_artifact", "swap_nvfp4_linears"]
