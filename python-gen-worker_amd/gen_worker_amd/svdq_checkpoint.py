"""nunchaku SVDQuant int4 checkpoints -> the int4-g64 modules, and swapping them into a denoiser.

The reference decodes nunchaku's "v1 single-file" svdq packaging for the nvfp4
variant (``src/gen_worker/models/svdq_layout.py``) and refuses int4
(``models/svdq.py:30-37``). An int4 svdq checkpoint stores the same tensors
with int4 arithmetic:

* ``qweight`` int8 [out, in/2]: two's-complement int4 codes in deepcompressor's
  mma.sync m16n8k64 fragment interleave, the same interleave the nvfp4 lane
  reads (``svdq_layout.py:11-13``, ``:87-107``): one int32 word holds 8 codes
  of one row (consecutive k), words ordered by (128-row tile, 64-column tile,
  16-row pack, row lane, k lane, row half, k half);
* ``wscales`` fp16 / bf16 [in/64, out]: group-64 scales in deepcompressor's
  ``pack_scale`` order (the per-channel vector swizzle of ``svdq_layout.py:
  128-137`` with the group as an extra dimension): per 128 output rows and
  group, the rows in the order (16-row lane group, 2-row pair, 8-row half,
  row in pair);
* ``smooth_factor`` [in] and ``bias`` [out]: ``pack_scale`` vectors;
  ``wcscales`` / ``wtscale`` (an optional second-level scale);
* ``proj_down`` [in, rank] and ``proj_up`` [out, rank]: ``pack_lowrank_weight``
  16 x 16 packs (``svdq_layout.py:140-161``); proj_down is applied to the RAW
  activation (the exporter pre-divided it by the smoothing factors). An
  artifact whose ``__metadata__`` declares ``lowrank_quant`` = int8 / fp8_e4m3
  stores the two factors plain row-major in that dtype with fp32 scales per
  32-block (``proj_down_scale`` [in/32, rank], ``proj_up_scale`` [out,
  rank/32]; ``svdq_layout.py:34-38``, ``:261-298``), decoded to bf16.

``decode_int4_linear`` returns the logical (row-major) tensors, ``split_decoded``
splits nunchaku's fused projections (``to_qkv`` -> ``to_q``/``to_k``/``to_v``,
``svdq_layout.py:441-470``) in that domain, and ``swap_svdq_linears`` /
``plan_targets`` (``models/svdq_native.py:239-321``) replace a model's
``nn.Linear`` modules with ``SvdqW4A4Linear`` in the qualified int4 lane (or a
folded dense Linear in the dense lane and where the kernel contract does not
hold). AWQ W4A16 modulation layers go through
``swap_awq_linears`` with the exporter's adaLN split count
(``models/svdq_native.py:324-338``). ``load_svdq_checkpoint`` reads a
safetensors file into a caller-built module skeleton (the reference builds
the stock diffusers class, which this environment does not ship). The fp4
packaging the reference serves (e4m3 micro-scales per 16 inputs) decodes
through ``svdq_fp4`` into the same logical domain and the same swap.

The interleaves are formats fixed by the checkpoints; the functions here
compute them independently (the oracle restates the forward packers with
explicit index arithmetic and the tests check one against the other).
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, replace
from typing import Any, Dict, Optional, Sequence

import torch
import torch.nn as nn
from torch import Tensor

logger = logging.getLogger(__name__)

GROUP = 64
_TILE_N, _TILE_K = 128, 64          # fragment tile of the weight interleave
_LR_PACK = 16                       # low-rank 16 x 16 packs

# weight interleave: codes [n, k] viewed as
#   (n_tile, n_pack 8, n_half 2, n_lane 8, k_tile, k_half 2, k_lane 4, k_reg 8)
# and stored in the order (n_tile, k_tile, n_pack, n_lane, k_lane, n_half, k_half, k_reg)
_W_VIEW = lambda n, k: (n // _TILE_N, 8, 2, 8, k // _TILE_K, 2, 4, 8)  # noqa: E731
_W_ORDER = (0, 4, 1, 3, 6, 2, 5, 7)
# scale / vector order: rows [n] of one group viewed as (block 128, lane-group 8, pair 2, lane 4, row 2)
# and stored in the order (block, group, lane-group, lane, pair, row)
_LR_ORDER = (0, 1, 3, 6, 2, 5, 4, 7)  # (c_pack, r_pack, n_lane, k_lane, n_half, k_half, n_reg, k_reg)

_FUSED_SPLITS: dict[str, tuple[str, ...]] = {
    "to_qkv": ("to_q", "to_k", "to_v"),
    "add_qkv_proj": ("add_q_proj", "add_k_proj", "add_v_proj"),
    "qkv_proj": ("q_proj", "k_proj", "v_proj"),
}
_ADANORM_SPLITS: dict[tuple[str, str], int] = {
    ("QwenImageTransformer2DModel", "img_mod.1"): 6,
    ("QwenImageTransformer2DModel", "txt_mod.1"): 6,
}


class SvdqLayoutError(ValueError):
    """A checkpoint layout this decoder does not understand (never guessed around)."""


def _inverse(order: Sequence[int]) -> tuple[int, ...]:
    inv = [0] * len(order)
    for i, p in enumerate(order):
        inv[p] = i
    return tuple(inv)


# ---------------------------------------------------------------------------
# interleaves
# ---------------------------------------------------------------------------

def unpack_qweight(qweight: Tensor, out_features: int, in_features: int) -> Tensor:
    """nunchaku ``qweight`` int8 [out, in/2] -> nibble codes uint8 [out, in] (two's-complement int4 nibbles)."""
    n, k = int(out_features), int(in_features)
    if n % _TILE_N or k % (2 * _TILE_K):
        raise SvdqLayoutError(f"svdq qweight [{n}, {k}] is not a multiple of the fragment tile "
                              f"({_TILE_N} x {2 * _TILE_K})")
    if tuple(qweight.shape) != (n, k // 2):
        raise SvdqLayoutError(f"svdq qweight shape {tuple(qweight.shape)} != {(n, k // 2)}")
    words = qweight.contiguous().view(torch.int32).reshape(-1)
    nib = (words.unsqueeze(-1) >> torch.arange(0, 32, 4, dtype=torch.int32, device=words.device)) & 0xF
    view = _W_VIEW(n, k)
    stored = nib.reshape(tuple(view[i] for i in _W_ORDER))
    return stored.permute(*_inverse(_W_ORDER)).reshape(n, k).to(torch.uint8)


def pack_qweight(codes: Tensor) -> Tensor:
    """Nibble codes [out, in] (values 0..15) -> nunchaku ``qweight`` int8 [out, in/2]."""
    n, k = int(codes.shape[0]), int(codes.shape[1])
    if n % _TILE_N or k % (2 * _TILE_K):
        raise SvdqLayoutError(f"svdq codes [{n}, {k}] are not a multiple of the fragment tile")
    c = (codes.to(torch.int32) & 0xF).reshape(_W_VIEW(n, k)).permute(*_W_ORDER)
    words = (c << torch.arange(0, 32, 4, dtype=torch.int32, device=c.device)).sum(dim=-1, dtype=torch.int32)
    return words.contiguous().view(torch.int8).reshape(n, k // 2)


def _scale_view(n: int, groups: int) -> tuple[int, ...]:
    return (n // 128, groups, 8, 4, 2, 2)   # stored order: (block, group, lane-group, lane, pair, row)


def unpack_group_scales(wscales: Tensor, out_features: int, in_features: int, group: int = GROUP) -> Tensor:
    """``pack_scale`` grid [in/group, out] -> row-major [out, in/group]."""
    n, g = int(out_features), int(in_features) // group
    if n % 128 or int(in_features) % group:
        raise SvdqLayoutError(f"svdq group scales for [{n}, {in_features}] break the pack (out % 128, in % {group})")
    if tuple(wscales.shape) != (g, n):
        raise SvdqLayoutError(f"svdq wscales shape {tuple(wscales.shape)} != {(g, n)}")
    s = wscales.contiguous().reshape(_scale_view(n, g))          # (block, group, a, c, b, d)
    s = s.permute(0, 2, 4, 3, 5, 1)                              # (block, a, b, c, d, group): row = 128 blk + 16a + 8b + 2c + d
    return s.reshape(n, g).contiguous()


def pack_group_scales(scales: Tensor) -> Tensor:
    """Row-major [out, groups] -> the ``pack_scale`` grid [groups, out]."""
    n, g = int(scales.shape[0]), int(scales.shape[1])
    if n % 128:
        raise SvdqLayoutError(f"svdq scale rows {n} are not a multiple of 128")
    s = scales.reshape(n // 128, 8, 2, 4, 2, g).permute(0, 5, 1, 3, 2, 4)
    return s.contiguous().reshape(g, n)


def unpack_vector(vec: Tensor, n: int) -> Tensor:
    """A ``pack_scale`` vector (one group) -> row-major [n]."""
    return unpack_group_scales(vec.reshape(1, -1), n, GROUP).reshape(n)


def pack_vector(vec: Tensor, n: int) -> Tensor:
    return pack_group_scales(vec.reshape(int(n), 1)).reshape(int(n))


def unpack_lowrank(weight: Tensor, *, down: bool) -> Tensor:
    """Stored ``proj_down`` [in, rank] -> [in, rank] row-major; stored ``proj_up`` [out, rank] -> [out, rank]."""
    c, r = int(weight.shape[0]), int(weight.shape[1])
    if c % _LR_PACK or r % _LR_PACK:
        raise SvdqLayoutError(f"svdq low-rank factor [{c}, {r}] breaks the 16 x 16 pack")
    w = weight.contiguous().reshape(c // 16, r // 16, 8, 4, 2, 2, 1, 2)
    w = w.permute(*_inverse(_LR_ORDER)).reshape(c // 16, r // 16, 16, 16)   # (cp, rp, i_n, i_k)
    if down:   # i_n runs over rank, i_k over the input
        return w.permute(0, 3, 1, 2).reshape(c, r).contiguous()
    return w.permute(0, 2, 1, 3).reshape(c, r).contiguous()   # i_n over the output, i_k over rank


def pack_lowrank(weight: Tensor, *, down: bool) -> Tensor:
    """Row-major [in, rank] (down) / [out, rank] (up) -> nunchaku's stored form (same shape)."""
    c, r = int(weight.shape[0]), int(weight.shape[1])
    if c % _LR_PACK or r % _LR_PACK:
        raise SvdqLayoutError(f"svdq low-rank factor [{c}, {r}] breaks the 16 x 16 pack")
    w = weight.reshape(c // 16, 16, r // 16, 16)
    w = w.permute(0, 2, 3, 1) if down else w.permute(0, 2, 1, 3)      # (cp, rp, i_n, i_k)
    w = w.reshape(c // 16, r // 16, 2, 8, 1, 2, 4, 2).permute(*_LR_ORDER)
    return w.contiguous().reshape(c, r)


# ---------------------------------------------------------------------------
# decoded linears
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class DecodedInt4Linear:
    """One int4 svdq linear in the logical domain: ``codes`` uint8 [out, in] two's-complement nibbles,
    ``scales`` fp16 [out, in/64], ``second`` fp32 [out] / [1] or None, ``proj_down`` [in, rank] and
    ``proj_up`` [out, rank] bf16, ``smooth_factor`` [in] and ``bias`` [out] bf16 (or None)."""

    out_features: int
    in_features: int
    codes: Tensor
    scales: Tensor
    second: Optional[Tensor] = None
    rank: int = 0
    proj_down: Optional[Tensor] = None
    proj_up: Optional[Tensor] = None
    smooth_factor: Optional[Tensor] = None
    bias: Optional[Tensor] = None


def is_int4_svdq_linear(tensors: dict[str, Tensor]) -> bool:
    """An int4 svdq linear stores 16-bit group-64 scales (the nvfp4 variant: e4m3 group-16 scales)."""
    ws = tensors.get("wscales")
    return "qweight" in tensors and ws is not None and ws.dtype in (torch.float16, torch.bfloat16) \
        and "wzeros" not in tensors


def _exact_fp16(t: Tensor, what: str) -> Tensor:
    h = t.to(torch.float16)
    if not torch.equal(h.float(), t.float()):
        raise SvdqLayoutError(f"{what} is not exactly representable in fp16 (the int4 lane's scale dtype)")
    return h


# Quantized low-rank branch (an artifact's ``__metadata__["lowrank_quant"]``, ``models/svdq_layout.py:34-38``):
# proj_down [in, rank] / proj_up [out, rank] stored PLAIN row-major as int8 or fp8 e4m3, with fp32 scales per
# block of 32 along each factor's contraction dimension: proj_down_scale [in/32, rank], proj_up_scale
# [out, rank/32]; the factor is RN_bf16(code * scale).
LOWRANK_QUANT_KEY = "lowrank_quant"
LOWRANK_SCHEMES = {"int8": torch.int8, "fp8_e4m3": torch.float8_e4m3fn}
LOWRANK_BLOCK = 32


def _lowrank_scheme(t: Tensor) -> str:
    for name, dt in LOWRANK_SCHEMES.items():
        if t.dtype == dt:
            return name
    return "bf16"


def dequantize_lowrank_factor(q: Tensor, scale: Tensor, *, along_rows: bool) -> Tensor:
    """bf16 factor = RN_bf16(code * scale), the scale of each block of 32 along the rows (proj_down: its
    input dimension) or along the columns (proj_up: the rank)."""
    rows, cols = int(q.shape[0]), int(q.shape[1])
    n = rows if along_rows else cols
    if n % LOWRANK_BLOCK:
        raise SvdqLayoutError(f"a quantized low-rank factor [{rows}, {cols}] needs its blocked dimension to be a "
                              f"multiple of {LOWRANK_BLOCK}")
    want = (n // LOWRANK_BLOCK, cols) if along_rows else (rows, n // LOWRANK_BLOCK)
    if tuple(scale.shape) != want:
        raise SvdqLayoutError(f"low-rank block scales {tuple(scale.shape)}: expected {want} for a [{rows}, {cols}] "
                              f"factor")
    per_elem = scale.float().repeat_interleave(LOWRANK_BLOCK, dim=0 if along_rows else 1)
    return (q.float() * per_elem).to(torch.bfloat16)


def quantize_lowrank_factor(w: Tensor, scheme: str, *, along_rows: bool) -> tuple[Tensor, Tensor]:
    """Producer of the quantized low-rank format (for synthetic checkpoints): per block of 32, scale =
    max(absmax / qmax, 1e-12) (qmax 127 for int8, 448 for e4m3), codes = round-to-nearest-even clamped
    (int8) or the e4m3 cast of the scaled value (``models/svdq_layout.py:261-275``)."""
    if scheme not in LOWRANK_SCHEMES:
        raise SvdqLayoutError(f"unknown low-rank scheme {scheme!r} (known: {', '.join(LOWRANK_SCHEMES)})")
    w32 = w.float()
    dim = 0 if along_rows else 1
    n = int(w32.shape[dim])
    if n % LOWRANK_BLOCK:
        raise SvdqLayoutError(f"dimension {n} is not a multiple of {LOWRANK_BLOCK}")
    blocks = w32.reshape(n // LOWRANK_BLOCK, LOWRANK_BLOCK, -1) if along_rows else \
        w32.reshape(w32.shape[0], n // LOWRANK_BLOCK, LOWRANK_BLOCK)
    qmax = 127.0 if scheme == "int8" else 448.0
    scale = (blocks.abs().amax(dim=1 if along_rows else 2) / qmax).clamp(min=1e-12)
    scaled = w32 / scale.repeat_interleave(LOWRANK_BLOCK, dim=dim)
    if scheme == "int8":
        q = torch.round(scaled).clamp(-127, 127).to(torch.int8)
    else:
        q = scaled.clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale.float()


def _decode_lowrank(down: Tensor, up: Tensor, tensors: dict[str, Tensor], n: int, k: int,
                    declared: Optional[str]) -> tuple[Tensor, Tensor, int]:
    """(proj_down bf16 [k, rank], proj_up bf16 [n, rank], rank) from either packaging of the branch."""
    scheme = _lowrank_scheme(down)
    if _lowrank_scheme(up) != scheme:
        raise SvdqLayoutError(f"proj_down is {down.dtype} but proj_up is {up.dtype}: one scheme per branch")
    if declared is not None and declared not in ("bf16",) + tuple(LOWRANK_SCHEMES):
        raise SvdqLayoutError(f"the artifact declares {LOWRANK_QUANT_KEY}={declared!r}, not one of bf16, "
                              f"{', '.join(LOWRANK_SCHEMES)}")
    if declared is not None and declared != scheme:
        raise SvdqLayoutError(f"the artifact declares {LOWRANK_QUANT_KEY}={declared!r} but the branch is stored "
                              f"as {scheme}")
    rank = int(down.shape[1])
    if int(down.shape[0]) != k or tuple(up.shape) != (n, rank):
        raise SvdqLayoutError(f"low-rank factors {tuple(down.shape)} / {tuple(up.shape)} do not match [{n}, {k}]")
    has_scales = "proj_down_scale" in tensors or "proj_up_scale" in tensors
    if scheme == "bf16":
        if has_scales:
            raise SvdqLayoutError("low-rank block scales are present but the factors are not stored quantized")
        if down.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise SvdqLayoutError(f"low-rank branch stored as {down.dtype}: not a 16/32-bit or int8 / fp8 factor")
        return unpack_lowrank(down, down=True).to(torch.bfloat16), unpack_lowrank(up, down=False).to(
            torch.bfloat16), rank
    for key in ("proj_down_scale", "proj_up_scale"):
        if key not in tensors:
            raise SvdqLayoutError(f"the {scheme} low-rank branch has no {key}")
    return (dequantize_lowrank_factor(down, tensors["proj_down_scale"], along_rows=True),
            dequantize_lowrank_factor(up, tensors["proj_up_scale"], along_rows=False), rank)


def decode_int4_linear(tensors: dict[str, Tensor], out_features: int, in_features: int, *,
                       lowrank_quant: Optional[str] = "bf16") -> DecodedInt4Linear:
    """One int4 svdq linear's stored tensors -> :class:`DecodedInt4Linear` (``decode_linear``,
    ``models/svdq_layout.py:366-434``, with int4 group-64 arithmetic); ``lowrank_quant`` is the artifact's
    declared low-rank scheme: "bf16" when the artifact declares none (the reference's default,
    ``models/svdq_native.py:376``), so quantized factors that were not declared are refused; None accepts
    whatever the factors' dtype says."""
    missing = [k for k in ("qweight", "wscales") if k not in tensors]
    if missing:
        raise SvdqLayoutError(f"not an svdq W4A4 linear (missing {missing})")
    if not is_int4_svdq_linear(tensors):
        raise SvdqLayoutError(f"wscales of dtype {tensors['wscales'].dtype}: not an int4 group-64 svdq linear "
                              f"(the nvfp4 packaging stores e4m3 group-16 scales)")
    n, k = int(out_features), int(in_features)
    codes = unpack_qweight(tensors["qweight"], n, k)
    scales = _exact_fp16(unpack_group_scales(tensors["wscales"], n, k), "wscales")
    second = None
    if "wcscales" in tensors:
        if int(tensors["wcscales"].numel()) != n:
            raise SvdqLayoutError(f"wcscales numel {int(tensors['wcscales'].numel())} != out_features {n}")
        second = unpack_vector(tensors["wcscales"].float().reshape(-1), n)
    elif "wtscale" in tensors:
        second = tensors["wtscale"].float().reshape(1)
    down, up = tensors.get("proj_down"), tensors.get("proj_up")
    if (down is None) != (up is None):
        raise SvdqLayoutError("svdq linear has only one half of the low-rank branch")
    rank = 0
    if down is not None:
        down, up, rank = _decode_lowrank(down, up, tensors, n, k, lowrank_quant)
    smooth = tensors.get("smooth_factor")
    if smooth is not None:
        smooth = unpack_vector(smooth.reshape(-1), k).to(torch.bfloat16)
    bias = tensors.get("bias")
    if bias is not None:
        bias = unpack_vector(bias.reshape(-1), n).to(torch.bfloat16)
    return DecodedInt4Linear(n, k, codes, scales, second, rank, down, up, smooth, bias)


def split_decoded(dec: DecodedInt4Linear, sections: Sequence[int]) -> tuple[DecodedInt4Linear, ...]:
    """Split a fused projection along the output dim (``models/svdq_layout.py:441-470``); the input-side
    tensors (smoothing, proj_down) are shared."""
    total = sum(int(s) for s in sections)
    if total != dec.out_features:
        raise SvdqLayoutError(f"split sections {tuple(sections)} sum to {total}, not out_features "
                              f"{dec.out_features}")
    out, a = [], 0
    for size in (int(s) for s in sections):
        b = a + size
        per_channel = dec.second is not None and dec.second.numel() > 1
        out.append(replace(dec, out_features=size, codes=dec.codes[a:b].contiguous(),
                           scales=dec.scales[a:b].contiguous(),
                           second=dec.second[a:b].contiguous() if per_channel else dec.second,
                           proj_up=dec.proj_up[a:b].contiguous() if dec.proj_up is not None else None,
                           bias=dec.bias[a:b].contiguous() if dec.bias is not None else None))
        a = b
    return tuple(out)


def dequantize_decoded(dec: DecodedInt4Linear) -> Tensor:
    """fp32 [out, in] = signed code * scale (* second): the 4-bit branch's weight (an fp4 linear: e2m1 code *
    e4m3 micro-scale * second)."""
    from .svdq_fp4 import DecodedFp4Linear, dequantize_fp4_decoded

    if isinstance(dec, DecodedFp4Linear):
        return dequantize_fp4_decoded(dec)
    c = dec.codes.to(torch.int16)
    c = torch.where(c >= 8, c - 16, c).float()
    w = (c.reshape(dec.out_features, -1, GROUP) * dec.scales.float().unsqueeze(-1)).reshape(dec.out_features, -1)
    if dec.second is not None:
        w = w * dec.second.float().reshape(-1, 1)
    return w


def fold_decoded(dec: DecodedInt4Linear, *, compute_dtype=torch.bfloat16, device=None) -> nn.Linear:
    """The dense lane (``fold_to_dense``, ``models/svdq_native.py:200-221``): one Linear with
    ``W_eff = deq(W) / smooth + up @ down^T`` for shapes the kernels do not take."""
    w = dequantize_decoded(dec)
    if dec.smooth_factor is not None:
        w = w / dec.smooth_factor.float().reshape(1, -1)
    if dec.rank:
        w = w + dec.proj_up.float() @ dec.proj_down.float().t()
    lin = nn.Linear(dec.in_features, dec.out_features, bias=dec.bias is not None, dtype=compute_dtype,
                    device=device)
    with torch.no_grad():
        lin.weight.copy_(w.to(compute_dtype))
        if dec.bias is not None:
            lin.bias.copy_(dec.bias.to(compute_dtype))
    lin.requires_grad_(False)
    return lin


def build_module(dec: DecodedInt4Linear, *, device: Any = "cuda", lane: Optional[str] = None,
                 fp4_mode: Optional[str] = None) -> nn.Module:
    """The device module for one decoded linear: ``SvdqW4A4Linear`` in the int4 lane when the kernel contract
    holds, else the folded dense Linear. ``lane`` None takes the process's qualified lane
    (``qualify.resolve_lane``; the reference decides its mode once, ``models/svdq_native.py:283-286``). An fp4
    linear goes by ``fp4_mode`` (``svdq_fp4.build_fp4_module``)."""
    from .qualify import resolve_lane
    from .svdq import build_svdq_w4a4_linear, fused_shape_supported
    from .svdq_fp4 import DecodedFp4Linear, build_fp4_module

    if isinstance(dec, DecodedFp4Linear):
        return build_fp4_module(dec, device=device, mode=fp4_mode)

    if resolve_lane(lane) != "int4" or not fused_shape_supported(dec.out_features, dec.in_features, dec.rank):
        return fold_decoded(dec, device=device)
    packed = (dec.codes[:, 0::2] & 0xF) | ((dec.codes[:, 1::2] & 0xF) << 4)
    return build_svdq_w4a4_linear(qweight=packed, wscales=dec.scales, smooth=dec.smooth_factor,
                                  proj_down=dec.proj_down if dec.rank else None,
                                  proj_up=dec.proj_up if dec.rank else None, bias=dec.bias,
                                  second=dec.second, device=device)


# ---------------------------------------------------------------------------
# swapping into a model: every replacement is resolved and checked against the model first, then applied,
# so a checkpoint that does not fit leaves the model untouched
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class SwapTarget:
    """One ``nn.Linear`` of the model that a checkpoint linear, or one part of a fused one, replaces."""

    path: str
    in_features: int
    out_features: int


def _linear_index(model: nn.Module) -> Dict[str, nn.Linear]:
    return {name: mod for name, mod in model.named_modules() if isinstance(mod, nn.Linear)}


def _replace(model: nn.Module, path: str, new: nn.Module) -> None:
    head, _, leaf = path.rpartition(".")
    setattr(model.get_submodule(head) if head else model, leaf, new)


def _resolve_targets(index: Dict[str, nn.Linear], prefix: str, model_name: str) -> tuple[SwapTarget, ...]:
    """The Linear named ``prefix``, or the Linears a fused projection name stands for (``to_qkv`` ->
    ``to_q``, ``to_k``, ``to_v`` beside it)."""
    lin = index.get(prefix)
    if lin is not None:
        return (SwapTarget(prefix, int(lin.in_features), int(lin.out_features)),)
    head, _, leaf = prefix.rpartition(".")
    parts = _FUSED_SPLITS.get(leaf)
    if parts is None:
        raise SvdqLayoutError(f"{prefix!r}: {model_name} has no nn.Linear of this name and {leaf!r} is not a fused "
                              f"projection this loader splits (it splits: {', '.join(sorted(_FUSED_SPLITS))})")
    paths = [f"{head}.{p}" if head else p for p in parts]
    missing = [p for p in paths if p not in index]
    if missing:
        raise SvdqLayoutError(f"{prefix!r} splits into {', '.join(paths)}, but {model_name} has no nn.Linear at "
                              f"{', '.join(missing)}")
    return tuple(SwapTarget(p, int(index[p].in_features), int(index[p].out_features)) for p in paths)


def plan_targets(model: nn.Module, prefix: str) -> tuple[tuple[str, int], ...]:
    """(path, out_features) of each Linear one checkpoint linear replaces (the reference's ``plan_targets``,
    ``models/svdq_native.py:239-267``, answers the same question)."""
    return tuple((t.path, t.out_features) for t in _resolve_targets(_linear_index(model), prefix,
                                                                     type(model).__name__))


def swap_svdq_linears(model: nn.Module, decoded: Dict[str, DecodedInt4Linear], *, device: Any = "cuda",
                      lane: Optional[str] = None, fp4_mode: Optional[str] = None) -> dict:
    """Install the checkpoint's svdq linears in ``model`` (the role of the reference's ``swap_svdq_linears``,
    ``models/svdq_native.py:270-321``): fused projections are split in the decoded domain, every piece must
    match the shape of the Linear it replaces, and each int4 piece becomes ``SvdqW4A4Linear`` in the int4 lane
    (the process's qualified lane unless ``lane`` says otherwise) or a folded dense Linear; each fp4 piece
    becomes ``SvdqFp4Linear`` in the blockwise ``fp4_mode`` or a folded Linear. Returns counts and the modes
    used."""
    from .qualify import resolve_lane
    from .svdq_fp4 import SvdqFp4Linear, resolve_fp4_mode

    index = _linear_index(model)
    name = type(model).__name__
    plan: list[tuple[SwapTarget, DecodedInt4Linear]] = []
    for prefix in sorted(decoded):
        dec = decoded[prefix]
        targets = _resolve_targets(index, prefix, name)
        pieces = (dec,) if len(targets) == 1 else split_decoded(dec, tuple(t.out_features for t in targets))
        for t, piece in zip(targets, pieces):
            if (piece.out_features, piece.in_features) != (t.out_features, t.in_features):
                raise SvdqLayoutError(f"{prefix!r} -> {t.path!r}: the checkpoint holds [{piece.out_features}, "
                                      f"{piece.in_features}], the model's nn.Linear is [{t.out_features}, "
                                      f"{t.in_features}]")
            plan.append((t, piece))
    chosen, fp4_chosen = resolve_lane(lane), resolve_fp4_mode(fp4_mode)
    counts: dict = {"prefixes": len(decoded), "linears": len(plan), "int4": 0, "blockwise": 0, "dense": 0,
                    "lane": chosen, "fp4_mode": fp4_chosen}
    for t, piece in plan:
        new = build_module(piece, device=device, lane=chosen, fp4_mode=fp4_chosen)
        kind = "dense" if isinstance(new, nn.Linear) else "blockwise" if isinstance(new, SvdqFp4Linear) else "int4"
        counts[kind] += 1
        _replace(model, t.path, new)
    logger.info("svdq swap (int4 lane %s, fp4 mode %s): %d checkpoint linears -> %d modules (%d int4, %d fp4 "
                "blockwise, %d dense)", chosen, fp4_chosen, counts["prefixes"], counts["linears"], counts["int4"],
                counts["blockwise"], counts["dense"])
    return counts


def adanorm_splits_for(model_class: str, prefix: str) -> int:
    """adaLN split count of one AWQ modulation layer from the verified table, matched on the longest tail of
    ``prefix`` (whole path components); anything else is refused, since a wrong count scrambles the
    modulation without any error (the reference keeps the same rule, ``models/svdq_native.py:324-338``)."""
    parts = prefix.split(".")
    for width in range(len(parts), 0, -1):
        n = _ADANORM_SPLITS.get((model_class, ".".join(parts[-width:])))
        if n is not None:
            return n
    raise SvdqLayoutError(f"{prefix!r} in {model_class or 'an unnamed model class'}: no verified adaLN split "
                          f"count; give it as adanorm_splits={{{prefix!r}: n}}")


def swap_awq_linears(model: nn.Module, layers: Dict[str, dict], *, model_class: str = "",
                     adanorm_splits: Optional[Dict[str, int]] = None, device: Any = "cuda") -> int:
    """Replace the AWQ W4A16 modulation Linears with packed modules (``models/svdq_native.py:414-436``)."""
    from .awq import build_awq_packed_linear

    index = _linear_index(model)
    plan = []
    for prefix in sorted(layers):
        target = index.get(prefix)
        if target is None:
            raise SvdqLayoutError(f"AWQ layer {prefix!r}: {type(model).__name__} has no nn.Linear of this name")
        splits = (adanorm_splits or {}).get(prefix)
        plan.append((prefix, target, adanorm_splits_for(model_class, prefix) if splits is None else splits))
    for prefix, target, splits in plan:
        _replace(model, prefix, build_awq_packed_linear(layers[prefix], int(target.out_features),
                                                        int(target.in_features), adanorm_splits=splits,
                                                        device=device))
    return len(plan)


def _group_by_prefix(names) -> dict[str, list[str]]:
    groups: dict[str, list[str]] = {}
    for key in names:
        prefix, _, leaf = key.rpartition(".")
        groups.setdefault(prefix, []).append(leaf)
    return groups


def load_svdq_checkpoint(path, model: nn.Module, *, model_class: str = "",
                         adanorm_splits: Optional[Dict[str, int]] = None, device: Any = "cuda",
                         lane: Optional[str] = None, lowrank_quant: Optional[str] = "bf16",
                         fp4_mode: Optional[str] = None, precision: Optional[str] = None) -> dict:
    """Read an svdq safetensors file into ``model`` (a skeleton whose module names match the checkpoint's;
    ``load_svdq_native_denoiser``, ``models/svdq_native.py:366-467``): int4 linears swapped for
    ``SvdqW4A4Linear`` and fp4 linears for ``SvdqFp4Linear`` (or folded Linears, per lane / mode; fused
    projections split), AWQ modulation linears for ``AwqPackedLinear``, every other tensor copied into the
    parameter / buffer of that name. ``precision`` ("int4" / "fp4"), when given, is the artifact's declared
    weight precision, and every linear must be stored in it."""
    from safetensors import safe_open

    from .awq import is_awq_linear
    from .svdq_fp4 import decode_fp4_linear, is_fp4_svdq_linear

    counts = {"int4_prefixes": 0, "fp4_prefixes": 0, "awq": 0, "plain": 0}
    decoded: Dict[str, DecodedInt4Linear] = {}
    awq_layers: Dict[str, dict] = {}
    plain: Dict[str, Tensor] = {}
    with safe_open(str(path), framework="pt", device="cpu") as fh:
        for prefix, leaves in sorted(_group_by_prefix(fh.keys()).items()):
            tensors = {leaf: fh.get_tensor(f"{prefix}.{leaf}" if prefix else leaf) for leaf in leaves}
            if is_awq_linear(tensors):
                awq_layers[prefix] = tensors
            elif "qweight" in tensors:
                targets = _resolve_targets(_linear_index(model), prefix, type(model).__name__)
                stored = "fp4" if is_fp4_svdq_linear(tensors) else "int4"
                if precision is not None and stored != precision:
                    raise SvdqLayoutError(f"{prefix!r} is stored as svdq-{stored} in an artifact that declares "
                                          f"svdq-{precision}")
                decode = decode_fp4_linear if stored == "fp4" else decode_int4_linear
                decoded[prefix] = decode(tensors, sum(t.out_features for t in targets), targets[0].in_features,
                                         lowrank_quant=lowrank_quant)
            else:
                for leaf, t in tensors.items():
                    plain[f"{prefix}.{leaf}" if prefix else leaf] = t
    counts["awq"] = swap_awq_linears(model, awq_layers, model_class=model_class, adanorm_splits=adanorm_splits,
                                     device=device)
    counts.update(swap_svdq_linears(model, decoded, device=device, lane=lane, fp4_mode=fp4_mode))
    counts["fp4_prefixes"] = sum(1 for d in decoded.values() if not isinstance(d, DecodedInt4Linear))
    counts["int4_prefixes"] = len(decoded) - counts["fp4_prefixes"]
    state = dict(model.named_parameters())
    state.update(dict(model.named_buffers()))
    with torch.no_grad():
        for name, t in plain.items():
            if name not in state:
                raise SvdqLayoutError(f"checkpoint tensor {name!r} has no parameter or buffer in {type(model).__name__}")
            dst = state[name]
            if tuple(dst.shape) != tuple(t.shape):
                raise SvdqLayoutError(f"{name!r}: checkpoint shape {tuple(t.shape)} != model {tuple(dst.shape)}")
            if dst.is_meta:
                parent, _, leaf = name.rpartition(".")
                owner = model.get_submodule(parent) if parent else model
                new = t.to(device=device, dtype=dst.dtype)
                if isinstance(dst, nn.Parameter):
                    setattr(owner, leaf, nn.Parameter(new, requires_grad=False))
                else:
                    owner.register_buffer(leaf, new)
            else:
                dst.copy_(t.to(dst.dtype))
            counts["plain"] += 1
    return counts


load_svdq_int4_checkpoint = load_svdq_checkpoint   # the name callers of the int4-only loader use


__all__ = [
    "DecodedInt4Linear", "LOWRANK_QUANT_KEY", "LOWRANK_SCHEMES", "SvdqLayoutError", "SwapTarget",
    "adanorm_splits_for", "dequantize_lowrank_factor", "quantize_lowrank_factor", "build_module", "decode_int4_linear",
    "dequantize_decoded", "fold_decoded", "is_int4_svdq_linear", "load_svdq_checkpoint", "load_svdq_int4_checkpoint",
    "pack_group_scales",
    "pack_lowrank", "pack_qweight", "pack_vector", "plan_targets", "split_decoded", "swap_awq_linears",
    "swap_svdq_linears", "unpack_group_scales", "unpack_lowrank", "unpack_qweight", "unpack_vector",
]
