"""Whole-denoiser loading for the W8A8 lane.

The reference serves W8A8 checkpoints (``src/gen_worker/models/w8a8.py``) by scanning the shards' headers
for quantized layers (``detect_w8a8_artifacts``, ``:66-134``), materializing a denoiser skeleton with each
quantized ``nn.Linear`` swapped for its scaled-GEMM module or dequantized where it cannot run quantized
(``load_w8a8_denoiser``, ``:446-522``), swapping the quantized Linears of an already-built model
(``swap_w8a8_linears``, ``:589-690``), dequantizing a raw state dict (``sanitize_w8a8_state_dict``,
``:570-586``), and producing such a checkpoint data-free from a bf16 tree (``quantize_tree_w8a8``,
``:738-792``).

The tensor contract per quantized layer ``L``: ``L.weight`` [out, in] of an 8-bit dtype, ``L.weight_scale``
fp32 (one value, or one per output channel: [out] / [out, 1]) that dequantizes it (w = weight * scale),
optional ``L.input_scale`` (fp32 scalar, a static activation scale), the bias unquantized. A layer is
quantized exactly when ``L.weight_scale`` exists beside an 8-bit ``L.weight`` (header evidence, never name
lists). This build's GEMM is int8 (``Int8ScaledLinear``): ``I8`` weights run quantized in the branch the
process qualified (``qualify.w8a8_gemm_mode``: "rowwise" or "pertensor"); ``F8_E4M3`` weights (the
reference's own format, which int8 cannot hold exactly) and every layer the GEMM cannot take (not a plain
``nn.Linear``, in_features % 64, out_features % 16, or the dequant lane) are served as their dequantized
weight in the compute dtype: the same numbers, never a refusal. Tensors are read with safetensors only
(nothing is unpickled).
"""

from __future__ import annotations

import json
import logging
import shutil
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Callable, Dict, Iterable, Optional, Sequence

import torch
import torch.nn as nn
from torch import Tensor

logger = logging.getLogger(__name__)

AUX_SUFFIXES = (".weight_scale", ".input_scale")
K_ALIGN, N_ALIGN = 64, 16          # the int8 GEMM's contract (Int8ScaledLinear)
INT8_DTYPES = ("I8", "int8", "torch.int8")
FP8_DTYPES = ("F8_E4M3", "float8_e4m3fn", "torch.float8_e4m3fn")
W8A8_FLAVOR = "int8-w8a8"          # the producer's quant_scheme tag (the reference writes "fp8-w8a8")
INT8_MAX = 127.0


class W8a8CheckpointError(ValueError):
    """The checkpoint does not match the W8A8 contract or the model it is loaded into."""


@dataclass(frozen=True)
class W8a8Artifact:
    """The shards of a W8A8 checkpoint (``W8a8Artifact``, ``models/w8a8.py:46-51``, plus the weights' kind)."""

    files: tuple[Path, ...]
    quantized: tuple[str, ...]
    static_input_scales: bool
    fp8: tuple[str, ...] = ()       # the quantized layers whose weights are e4m3 (dequantized on load)


def _kind(dtype: Any) -> str:
    d = str(dtype)
    if d in INT8_DTYPES:
        return "int8"
    if d in FP8_DTYPES:
        return "fp8"
    return ""


def quantized_w8a8_layers(names: Iterable[str], dtype_of: Callable[[str], Any]) -> dict:
    """{layer: "int8" | "fp8"} for every ``L.weight_scale`` whose ``L.weight`` has an 8-bit dtype
    (``_quantized_layers``, ``models/w8a8.py:66-79``); ``dtype_of`` gives a safetensors dtype string or a torch
    dtype."""
    names = set(names)
    out = {}
    for key in names:
        if not key.endswith(".weight_scale"):
            continue
        layer = key[: -len(".weight_scale")]
        if f"{layer}.weight" in names:
            kind = _kind(dtype_of(f"{layer}.weight"))
            if kind:
                out[layer] = kind
    return dict(sorted(out.items()))


def scan_w8a8_artifact(files: Sequence[Any]) -> W8a8Artifact:
    """Read the shards' headers (no tensor data) and list the quantized layers; no quantized layer raises."""
    from safetensors import safe_open

    paths = tuple(Path(f) for f in files)
    dtypes: Dict[str, str] = {}
    for p in paths:
        with safe_open(str(p), framework="pt", device="cpu") as fh:
            for name in fh.keys():
                if name in dtypes:
                    raise W8a8CheckpointError(f"tensor {name!r} appears in more than one shard")
                dtypes[name] = fh.get_slice(name).get_dtype()
    layers = quantized_w8a8_layers(dtypes, dtypes.__getitem__)
    if not layers:
        raise W8a8CheckpointError(f"no W8A8 layer (8-bit weight + weight_scale) in {len(paths)} shard(s)")
    q = tuple(layers)
    return W8a8Artifact(paths, q, any(f"{n}.input_scale" in dtypes for n in q),
                        tuple(n for n, k in layers.items() if k == "fp8"))


def shard_files(root: Path | str) -> tuple[Path, ...]:
    """The weight shards under a snapshot folder: those an index names, then the other ``*.safetensors``, in
    each directory below ``root`` (hidden ones skipped) (``_root_weight_files``, ``models/w8a8.py:82-100``)."""
    root = Path(root)
    dirs = [root] + sorted(p for p in root.rglob("*") if p.is_dir()
                           and not any(part.startswith(".") for part in p.relative_to(root).parts))
    out: list[Path] = []
    for d in dirs:
        indexed: list[str] = []
        for idx in sorted(d.glob("*.safetensors.index.json")):
            try:
                indexed += [str(v) for v in (json.loads(idx.read_text("utf-8")).get("weight_map") or {}).values()]
            except (OSError, ValueError):
                continue
        out += [d / n for n in sorted(set(indexed)) if (d / n).is_file()]
        out += [p for p in sorted(d.glob("*.safetensors")) if p.is_file() and p.name not in set(indexed)]
    return tuple(dict.fromkeys(out))


def detect_w8a8_artifacts(model_path: Path | str) -> tuple[tuple[str, W8a8Artifact], ...]:
    """Every quantized denoiser of a snapshot as (component, artifact): with a ``model_index.json``, each
    denoiser folder (``svdq_artifact.DENOISER_DIRS`` order) holding quantized layers; otherwise the snapshot's
    own shards as component "" (``detect_w8a8_artifacts``, ``models/w8a8.py:103-128``)."""
    from .svdq_artifact import DENOISER_DIRS

    root = Path(model_path)
    if not root.is_dir():
        return ()
    found = []
    if (root / "model_index.json").exists():
        for comp in DENOISER_DIRS:
            files = tuple(sorted(p for p in (root / comp).glob("*.safetensors") if p.is_file())) \
                if (root / comp).is_dir() else ()
            if files:
                try:
                    found.append((comp, scan_w8a8_artifact(files)))
                except W8a8CheckpointError:
                    continue
        return tuple(found)
    files = shard_files(root)
    if files:
        try:
            found.append(("", scan_w8a8_artifact(files)))
        except W8a8CheckpointError:
            pass
    return tuple(found)


def scale_per_channel(scale: Tensor, out_features: int) -> Tensor:
    """``weight_scale`` (one value or one per output channel) -> fp32 [out, 1] (``_scale_2d``,
    ``models/w8a8.py:398-405``)."""
    s = scale.detach().float()
    if s.numel() == 1:
        return s.reshape(1, 1).expand(out_features, 1).contiguous()
    if s.numel() != out_features:
        raise W8a8CheckpointError(f"weight_scale has {s.numel()} values for {out_features} output channels")
    return s.reshape(out_features, 1).contiguous()


def dequantize_w8a8_tensor(weight: Tensor, weight_scale: Tensor) -> Tensor:
    """An 8-bit weight [out, in] and its scale -> float32 [out, in] = weight * scale (one rounding per element,
    as the reference's ``w.float() * _scale_2d(scale)``, ``models/w8a8.py:485-486``)."""
    if weight.dim() != 2 or not _kind(weight.dtype):
        raise W8a8CheckpointError(f"weight must be an 8-bit [out, in] tensor, got {weight.dtype} "
                                  f"{tuple(weight.shape)}")
    return weight.float() * scale_per_channel(weight_scale, int(weight.shape[0])).to(weight.device)


def sanitize_w8a8_state_dict(state_dict: Dict[str, Tensor], compute_dtype: torch.dtype = torch.bfloat16
                             ) -> Dict[str, Tensor]:
    """A raw state dict with every quantized layer's weight dequantized into ``compute_dtype`` and its scale
    tensors dropped; other tensors as given (``sanitize_w8a8_state_dict``, ``models/w8a8.py:570-586``)."""
    quantized = quantized_w8a8_layers(state_dict, lambda k: state_dict[k].dtype)
    out: Dict[str, Tensor] = {}
    for key, t in state_dict.items():
        layer = key[: -len(".weight")] if key.endswith(".weight") else None
        if layer is not None and layer in quantized:
            out[key] = dequantize_w8a8_tensor(t, state_dict[f"{layer}.weight_scale"]).to(compute_dtype)
        elif any(key.endswith(s) and key[: -len(s)] in quantized for s in AUX_SUFFIXES):
            continue
        else:
            out[key] = t
    return out


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
            raise W8a8CheckpointError(f"artifact tensor {name!r} missing from the shards")
        return fh.get_tensor(name)

    def layer(self, layer: str) -> Dict[str, Tensor]:
        return {f"{layer}{s}": self.get(f"{layer}{s}") for s in (".weight", ".bias") + AUX_SUFFIXES
                if f"{layer}{s}" in self.where}


def _module_at(model: nn.Module, path: str) -> tuple[nn.Module, str, Any]:
    parent_path, _, leaf = path.rpartition(".")
    try:
        parent = model.get_submodule(parent_path) if parent_path else model
        return parent, leaf, getattr(parent, leaf)
    except AttributeError as exc:
        raise W8a8CheckpointError(f"no module {path!r} in {type(model).__name__}") from exc


def _dequant_reason(old: Any, kind: str, out_f: int, in_f: int, mode: str) -> Optional[str]:
    """Why a layer is served dequantized (None: it runs on Int8ScaledLinear)."""
    if mode == "dequant":
        return "dequant_lane"
    if kind != "int8":
        return "fp8_weight"
    if type(old) is not nn.Linear:
        return "not_plain_linear"
    if in_f % K_ALIGN or out_f % N_ALIGN:
        return "dim_unaligned"
    return None


def _layer_bias(layer: str, target: str, tensors: Dict[str, Tensor], old: Any) -> Optional[Tensor]:
    """The layer's bias: the checkpoint's ``L.bias`` when the module has a bias, else the module's own when it
    is materialized. A checkpoint bias on a module without one, or a module bias that neither provides, raises
    (the reference's ``load_state_dict`` reports both as unexpected / missing keys)."""
    ckpt = tensors.get(f"{layer}.bias")
    mod_bias = getattr(old, "bias", None)
    if mod_bias is None:
        if ckpt is not None:
            raise W8a8CheckpointError(f"checkpoint has {layer}.bias but module {target!r} has no bias")
        return None
    if ckpt is not None:
        return ckpt
    if mod_bias.is_meta:
        raise W8a8CheckpointError(f"module {target!r} has a bias the checkpoint does not provide")
    return mod_bias.detach()


def swap_w8a8_linears(model: nn.Module, art: W8a8Artifact, *, key_map: Optional[Callable[[str], str]] = None,
                      device: Any = "cuda", mode: Optional[str] = None,
                      compute_dtype: torch.dtype = torch.bfloat16) -> dict:
    """Swap the artifact's quantized layers in an already-built ``model`` (``swap_w8a8_linears``): each plain,
    aligned ``nn.Linear`` with int8 weights becomes an ``Int8ScaledLinear`` in ``mode`` (default: the
    process's qualified branch, ``qualify.resolve_w8a8_mode``); every other keeps its module with the
    dequantized weight assigned. ``key_map`` maps an artifact layer name to the model's module path. Returns
    {"quantized", "swapped", "mode", "dequantized": {reason: count}}; a shape mismatch raises."""
    from .qualify import resolve_w8a8_mode
    from .w8a8 import build_int8_linear

    mode = resolve_w8a8_mode(mode)
    fp8 = set(art.fp8)
    reader = _ShardReader(art.files)
    counts: Dict[str, Any] = {"quantized": len(art.quantized), "swapped": 0, "mode": mode, "dequantized": {}}
    for layer in art.quantized:
        target = key_map(layer) if key_map is not None else layer
        parent, leaf, old = _module_at(model, target)
        tensors = reader.layer(layer)
        w = tensors[f"{layer}.weight"]
        out_f, in_f = int(w.shape[0]), int(w.shape[1])
        mod_shape = (getattr(old, "out_features", None), getattr(old, "in_features", None))
        if mod_shape != (out_f, in_f):
            raise W8a8CheckpointError(f"layer {layer!r} is [{out_f}, {in_f}] in the checkpoint, module {target!r} "
                                      f"is {list(mod_shape)}")
        bias = _layer_bias(layer, target, tensors, old)
        why = _dequant_reason(old, "fp8" if layer in fp8 else "int8", out_f, in_f, mode)
        scale = scale_per_channel(tensors[f"{layer}.weight_scale"], out_f)
        if why is None:
            new = build_int8_linear(qweight=w, weight_scale=scale,
                                    bias=bias.to(compute_dtype) if bias is not None else None,
                                    compute_dtype=compute_dtype, device=device,
                                    input_scale=tensors.get(f"{layer}.input_scale"), gemm_mode=mode)
            setattr(parent, leaf, new)
            counts["swapped"] += 1
        else:
            dense = dequantize_w8a8_tensor(w, scale).to(device=device, dtype=compute_dtype)
            old.weight = nn.Parameter(dense, requires_grad=False)
            if bias is not None:
                old.bias = nn.Parameter(bias.to(device=device, dtype=compute_dtype), requires_grad=False)
            counts["dequantized"][why] = counts["dequantized"].get(why, 0) + 1
    partial = {k: v for k, v in counts["dequantized"].items() if k != "dequant_lane"}
    if partial:
        logger.warning("w8a8 swap: %d/%d quantized layers on Int8ScaledLinear (%s), %s served dequantized",
                       counts["swapped"], counts["quantized"], mode,
                       ", ".join(f"{k}={v}" for k, v in sorted(partial.items())))
    return counts


def load_w8a8_denoiser(art: Any, model: nn.Module, *, key_map: Optional[Callable[[str], str]] = None,
                       device: Any = "cuda", mode: Optional[str] = None,
                       compute_dtype: torch.dtype = torch.bfloat16) -> dict:
    """Materialize ``model`` (a skeleton whose parameters may sit on the meta device) from a W8A8 checkpoint
    (``load_w8a8_denoiser``, ``models/w8a8.py:446-522``): the quantized layers through ``swap_w8a8_linears``,
    every other tensor assigned to the parameter or buffer of its name (floating tensors in
    ``compute_dtype``). A checkpoint tensor with no home, a shape mismatch, or a model tensor the checkpoint
    leaves unset raises. ``art``: a ``W8a8Artifact`` or the shard paths. Returns the swap counts plus
    {"plain": n}."""
    if not isinstance(art, W8a8Artifact):
        art = scan_w8a8_artifact(art if isinstance(art, (list, tuple)) else [art])
    counts = swap_w8a8_linears(model, art, key_map=key_map, device=device, mode=mode, compute_dtype=compute_dtype)
    claimed = set()
    for layer in art.quantized:
        claimed.update(f"{layer}{s}" for s in (".weight", ".bias") + AUX_SUFFIXES)
    reader = _ShardReader(art.files)
    homes = dict(model.named_parameters())
    homes.update(dict(model.named_buffers()))
    plain = 0
    with torch.no_grad():
        for name in reader.where:
            if name in claimed:
                continue
            prefix, _, leaf = name.rpartition(".")
            target = f"{key_map(prefix)}.{leaf}" if (key_map is not None and prefix) else name
            if target not in homes:
                raise W8a8CheckpointError(f"checkpoint tensor {name!r} has no parameter or buffer {target!r} in "
                                          f"{type(model).__name__}")
            t = reader.get(name)
            dst = homes[target]
            if tuple(dst.shape) != tuple(t.shape):
                raise W8a8CheckpointError(f"{name!r}: checkpoint shape {tuple(t.shape)} != model {tuple(dst.shape)}")
            if t.is_floating_point():
                t = t.to(compute_dtype)
            owner_path, _, leaf_name = target.rpartition(".")
            owner = model.get_submodule(owner_path) if owner_path else model
            if isinstance(dst, nn.Parameter):
                setattr(owner, leaf_name, nn.Parameter(t.to(device), requires_grad=False))
            else:
                owner.register_buffer(leaf_name, t.to(device))
            plain += 1
    missing = [n for n, p in list(model.named_parameters()) + list(model.named_buffers()) if p.is_meta]
    if missing:
        raise W8a8CheckpointError(f"the checkpoint leaves {len(missing)} model tensor(s) unset, e.g. {missing[:5]}")
    model.eval()
    counts["plain"] = plain
    return counts


def quantize_state_dict_w8a8(state_dict: Dict[str, Tensor], *, exclude: tuple[str, ...] = ("embed", "norm")
                             ) -> tuple[Dict[str, Tensor], int]:
    """The data-free producer's per-shard step (``quantize_tree_w8a8``, ``models/w8a8.py:762-786``, int8
    form): every floating 2-D ``L.weight`` with both dims % 16 and no ``exclude`` substring in ``L`` becomes
    int8 codes ``clamp(rne(w / s), -127, 127)`` with ``s = max(amax_row / 127, 1e-12)`` stored as
    ``L.weight_scale`` fp32 [out] (the producer ``quantize_weight_int8`` of the module); the rest is copied.
    Returns (tensors, layers quantized)."""
    from .w8a8 import quantize_weight_int8

    out: Dict[str, Tensor] = {}
    n = 0
    for name, t in state_dict.items():
        layer = name[: -len(".weight")] if name.endswith(".weight") else ""
        if (layer and t.dim() == 2 and t.is_floating_point() and t.dtype != torch.float8_e4m3fn
                and t.shape[0] % N_ALIGN == 0 and t.shape[1] % N_ALIGN == 0
                and not any(x in layer for x in exclude)):
            q, s = quantize_weight_int8(t)
            out[name] = q.contiguous()
            out[f"{layer}.weight_scale"] = s.reshape(-1).contiguous()
            n += 1
        else:
            out[name] = t
    return out, n


def quantize_tree_w8a8(src_tree: Path | str, out_tree: Path | str, *,
                       exclude: tuple[str, ...] = ("embed", "norm")) -> Path:
    """Copy a diffusers tree, rewriting its denoiser's shards through ``quantize_state_dict_w8a8`` and tagging
    the denoiser's config with its quantization (``quantize_tree_w8a8``, ``models/w8a8.py:738-792``)."""
    from safetensors.torch import load_file, save_file

    from .svdq_artifact import DENOISER_DIRS

    src, out = Path(src_tree), Path(out_tree)
    comp = next((c for c in DENOISER_DIRS if (src / c).is_dir()), None)
    if comp is None or not (src / "model_index.json").exists():
        raise W8a8CheckpointError(f"{src} is not a diffusers tree with a denoiser folder")
    if out.exists():
        shutil.rmtree(out)
    shutil.copytree(src, out, ignore=shutil.ignore_patterns("*.safetensors"))
    for f in sorted(src.rglob("*.safetensors")):
        rel = f.relative_to(src)
        dst = out / rel
        dst.parent.mkdir(parents=True, exist_ok=True)
        if rel.parts[0] != comp:
            shutil.copy2(f, dst)
            continue
        tensors, n = quantize_state_dict_w8a8(load_file(str(f)), exclude=exclude)
        save_file(tensors, str(dst), metadata={"quant_scheme": W8A8_FLAVOR})
        logger.info("w8a8 producer: %s, %d layers quantized", rel, n)
    cfg_path = out / comp / "config.json"
    cfg = json.loads(cfg_path.read_text("utf-8")) if cfg_path.exists() else {}
    cfg["quantization_config"] = {"quant_method": "gen_worker_amd", "quant_algo": "INT8"}
    cfg_path.write_text(json.dumps(cfg, indent=2))
    return out


__all__ = ["AUX_SUFFIXES", "K_ALIGN", "N_ALIGN", "W8A8_FLAVOR", "W8a8Artifact", "W8a8CheckpointError",
           "dequantize_w8a8_tensor", "detect_w8a8_artifacts", "load_w8a8_denoiser", "quantize_state_dict_w8a8",
           "quantize_tree_w8a8", "quantized_w8a8_layers", "sanitize_w8a8_state_dict", "scale_per_channel",
           "scan_w8a8_artifact", "shard_files", "swap_w8a8_linears"]
