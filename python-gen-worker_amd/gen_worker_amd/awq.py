"""AWQ W4A16 modulation layers (group-64 asymmetric uint4 weights, bf16 activations).

An svdq checkpoint keeps its adaLN modulation linears (``img_mod`` /
``txt_mod``, the timestep-embedding consumers, M = 1 token) as AWQ W4A16, not
W4A4 (``src/gen_worker/models/svdq_awq.py:1``). This module is the host side
of that lane on the HIP kernels of ``libgen_worker_amd.so``:

* the on-disk format (``models/svdq_awq.py``): ``qweight`` int32 [oc/4, ic/2]
  in the TinyChat nibble interleave (``unpack_w4x16`` / ``pack_w4x16``),
  ``wscales`` / ``wzeros`` bf16 [num_scale_rows, oc] (zero-padded rows; zeros
  pre-scaled and pre-negated, so w = code * s + z), and the exporter's adaLN
  transform (``adanorm_splits``: output rows interleaved and +1 folded into
  the bias of splits 1 and splits - 2);
* the packed-resident module ``AwqPackedLinear`` (``models/svdq_awq_packed.py:
  152-207``: weight uint8 [oc, ic/2], wscales / wzeros [oc, ic/64]) whose
  forward is the ``cozy_gen_worker::awq_w4a16_mm`` op, and
  ``build_awq_packed_linear`` from the on-disk tensors
  (``models/svdq_awq_packed.py:221-253``);
* ``decode_awq_linear``: the reference's any-hardware lane (a plain bf16
  ``nn.Linear`` holding the dequantized weight) and ``encode_awq_linear``,
  the exporter-layout producer used to synthesize inputs.

The TinyChat interleave and the adaLN transform are formats fixed by the
checkpoints, so the functions here compute exactly what the reference's
functions of the same names compute, written independently.
"""

from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn as nn
from torch import Tensor

GROUP_SIZE = 64
_SCALE_PACK = 8                     # scale rows are written in packs of 8 groups
_PACK_MULTIPLE = {32: 4, 64: 2}     # and the pack count rounded up to this multiple per group size


class AwqLayoutError(ValueError):
    """The AWQ tensors do not match the layout this decoder understands."""


class AwqPackedError(RuntimeError):
    """Typed packed-AWQ failure (contract mismatch; never a silent wrong result)."""


def awq_packed_supported(out_features: int, in_features: int) -> bool:
    """The packed lane's shape contract (``models/svdq_awq_packed.py:23-24``)."""
    return out_features % 16 == 0 and in_features % 128 == 0


def num_scale_rows(in_features: int, group_size: int) -> int:
    """Row count of the exporter's (padded) scale / zero grids (``models/svdq_awq.py:18-28``)."""
    if in_features % group_size:
        raise AwqLayoutError(f"in_features {in_features} not divisible by group size {group_size}")
    groups = in_features // group_size
    packs = -(-groups // _SCALE_PACK)
    mult = _PACK_MULTIPLE.get(group_size, 1)
    return -(-packs // mult) * mult * _SCALE_PACK


def _check_codes_shape(oc: int, ic: int) -> None:
    if oc % 4 or ic % 64:
        raise AwqLayoutError(f"AWQ W4A16 [{oc}, {ic}] needs oc % 4 == 0 and ic % 64 == 0")


def pack_w4x16(codes: Tensor) -> Tensor:
    """Codes [oc, ic] (0..15) -> TinyChat int32 [oc/4, ic/2] (``models/svdq_awq.py:140-151``).

    Per row, every 32-code block b becomes 8 int16 words, word j holding codes 32b + j, +8, +16, +24 in
    its four nibbles (lowest first); the words of 4 consecutive rows are then interleaved in 64-column
    units (16 words of row 4R, then of 4R+1, 4R+2, 4R+3), and word pairs read as int32."""
    oc, ic = int(codes.shape[0]), int(codes.shape[1])
    _check_codes_shape(oc, ic)
    c = codes.to(torch.int32).reshape(oc, ic // 32, 4, 8)  # [row, block, nibble, word]
    words = c[:, :, 0] | (c[:, :, 1] << 4) | (c[:, :, 2] << 8) | (c[:, :, 3] << 12)  # [row, block, 8]
    words = words.reshape(oc // 4, 4, ic // 64, 16).transpose(1, 2).reshape(oc // 4, ic)
    return words.to(torch.int16).view(torch.int32)


def unpack_w4x16(qweight: Tensor, out_features: int, in_features: int) -> Tensor:
    """TinyChat int32 [oc/4, ic/2] -> codes uint8 [oc, ic] (``models/svdq_awq.py:31-46``)."""
    oc, ic = int(out_features), int(in_features)
    _check_codes_shape(oc, ic)
    if tuple(qweight.shape) != (oc // 4, ic // 2):
        raise AwqLayoutError(f"AWQ qweight shape {tuple(qweight.shape)} != expected {(oc // 4, ic // 2)} "
                             f"for [{oc}, {ic}]")
    words = qweight.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF  # [oc/4, ic]
    words = words.reshape(oc // 4, ic // 64, 4, 16).transpose(1, 2).reshape(oc, ic // 32, 8)
    nibbles = torch.stack([(words >> (4 * i)) & 0xF for i in range(4)], dim=2)  # [row, block, nibble, word]
    return nibbles.reshape(oc, ic).to(torch.uint8)


def scales_and_zeros(wscales: Tensor, wzeros: Tensor, out_features: int,
                     in_features: int) -> tuple[Tensor, Tensor, int]:
    """Padded grids [rows, oc] -> (scale, zero) fp32 [oc, groups] and the group size
    (``models/svdq_awq.py:49-71``: the live groups are the leading rows with a nonzero scale)."""
    oc, ic = int(out_features), int(in_features)
    if int(wscales.shape[1]) != oc or tuple(wzeros.shape) != tuple(wscales.shape):
        raise AwqLayoutError(f"AWQ scale/zero grids {tuple(wscales.shape)}/{tuple(wzeros.shape)} do not match "
                             f"out_features {oc}")
    s = wscales.float()
    live = (s != 0).any(dim=1)
    ng = int(live.sum())
    if ng == 0 or not bool(live[:ng].all()):
        raise AwqLayoutError("AWQ wscales has zero rows before its last live row (not the padded layout)")
    if ic % ng:
        raise AwqLayoutError(f"in_features {ic} not divisible by {ng} live scale groups")
    gs = ic // ng
    if num_scale_rows(ic, gs) != int(wscales.shape[0]):
        raise AwqLayoutError(f"AWQ scale rows {int(wscales.shape[0])} != num_scale_rows({ic}, {gs}) = "
                             f"{num_scale_rows(ic, gs)}")
    return s[:ng].t().contiguous(), wzeros.float()[:ng].t().contiguous(), gs


def dequantize_w4x16(qweight: Tensor, wscales: Tensor, wzeros: Tensor, out_features: int,
                     in_features: int) -> Tensor:
    """AWQ tensors -> fp32 weight [oc, ic] = code * scale + zero (``models/svdq_awq.py:74-82``)."""
    codes = unpack_w4x16(qweight, out_features, in_features)
    scale, zero, gs = scales_and_zeros(wscales, wzeros, out_features, in_features)
    oc, ic = int(out_features), int(in_features)
    w = codes.float().reshape(oc, ic // gs, gs)
    return (w * scale.unsqueeze(-1) + zero.unsqueeze(-1)).reshape(oc, ic)


def _split_delta(splits: int, dtype, device) -> Tensor:
    d = torch.zeros(splits, dtype=dtype, device=device)
    d[1] = 1.0
    d[splits - 2] = 1.0
    return d


def apply_adanorm_splits(weight: Tensor, bias: Optional[Tensor], splits: int) -> tuple[Tensor, Optional[Tensor]]:
    """The exporter's adaLN transform (``models/svdq_awq.py:154-171``): stored row j * splits + s is
    original row s * (oc / splits) + j, and the bias of splits 1 and splits - 2 gains +1."""
    if splits <= 1:
        return weight, bias
    oc = int(weight.shape[0])
    if oc % splits:
        raise AwqLayoutError(f"out_features {oc} not divisible by adanorm_splits {splits}")
    if bias is None:
        raise AwqLayoutError("adanorm_splits > 1 needs a bias (adaLN folds 1 + scale into it)")
    per = oc // splits
    w = weight.reshape(splits, per, -1).transpose(0, 1).reshape(oc, -1)
    b = bias.reshape(splits, per) + _split_delta(splits, bias.dtype, bias.device).reshape(splits, 1)
    return w, b.transpose(0, 1).reshape(oc)


def undo_adanorm_splits(weight: Tensor, bias: Optional[Tensor], splits: int) -> tuple[Tensor, Optional[Tensor]]:
    """Inverse of :func:`apply_adanorm_splits` (``models/svdq_awq.py:85-103``)."""
    if splits <= 1:
        return weight, bias
    oc = int(weight.shape[0])
    if oc % splits:
        raise AwqLayoutError(f"out_features {oc} not divisible by adanorm_splits {splits}")
    per = oc // splits
    w = weight.reshape(per, splits, -1).transpose(0, 1).reshape(oc, -1)
    return w, (_undo_split_bias(bias, splits) if bias is not None else None)


def _undo_split_bias(bias: Tensor, splits: int) -> Tensor:
    oc = int(bias.numel())
    b = bias.float().reshape(oc // splits, splits).transpose(0, 1)
    b = b - _split_delta(splits, b.dtype, b.device).reshape(splits, 1)
    return b.reshape(oc)


def _undo_interleave_rows(oc: int, splits: int, device) -> Tensor:
    """Index of the stored row that holds original row i (original row s * per + j is stored at j * splits + s)."""
    per = oc // splits
    i = torch.arange(oc, device=device)
    return (i % per) * splits + i // per


def encode_awq_linear(weight: Tensor, bias: Optional[Tensor], *, group_size: int = GROUP_SIZE,
                      adanorm_splits: int = 1) -> dict[str, Tensor]:
    """One Linear -> the exporter-layout AWQ tensors (``models/svdq_awq.py:174-210``): per-group min/max
    over ``group_size`` inputs, scale = max((max - min) / 15, 1e-6), zero = (-min / scale) * scale,
    code = clamp(round((w + zero) / scale), 0, 15); grids zero-padded to ``num_scale_rows`` rows, zeros
    stored negated."""
    w = weight.detach().float()
    b = bias.detach().float() if bias is not None else None
    w, b = apply_adanorm_splits(w, b, int(adanorm_splits))
    oc, ic = int(w.shape[0]), int(w.shape[1])
    if ic % group_size:
        raise AwqLayoutError(f"in_features {ic} not divisible by group size {group_size}")
    ng = ic // group_size
    g = w.reshape(oc, ng, group_size)
    lo, hi = g.amin(dim=-1), g.amax(dim=-1)
    scale = ((hi - lo) / 15.0).clamp(min=1e-6)
    zero = (-lo / scale) * scale
    q = torch.round((g + zero.unsqueeze(-1)) / scale.unsqueeze(-1)).clamp(0.0, 15.0).reshape(oc, ic)
    rows = num_scale_rows(ic, group_size)
    wscales = torch.zeros(rows, oc, dtype=torch.bfloat16, device=w.device)
    wzeros = torch.zeros(rows, oc, dtype=torch.bfloat16, device=w.device)
    wscales[:ng] = scale.t().to(torch.bfloat16)
    wzeros[:ng] = (-zero).t().to(torch.bfloat16)
    out = {"qweight": pack_w4x16(q.to(torch.uint8)), "wscales": wscales, "wzeros": wzeros}
    if b is not None:
        out["bias"] = b.to(torch.bfloat16)
    return out


def is_awq_linear(tensors: dict[str, Any]) -> bool:
    """``wzeros`` tells AWQ W4A16 linears from the W4A4 svdq linears (``models/svdq_awq.py:132-134``)."""
    return "wzeros" in tensors and "qweight" in tensors


def decode_awq_linear(tensors: dict[str, Tensor], out_features: int, in_features: int, *,
                      adanorm_splits: int = 1, compute_dtype: Optional[torch.dtype] = None,
                      device=None) -> nn.Linear:
    """The reference's decode lane (``models/svdq_awq.py:106-129``): a plain ``nn.Linear`` in
    ``compute_dtype`` (bf16) holding the dequantized weight, adaLN transform undone."""
    missing = [k for k in ("qweight", "wscales", "wzeros") if k not in tensors]
    if missing:
        raise AwqLayoutError(f"not an AWQ W4A16 linear (missing {missing})")
    compute = compute_dtype or torch.bfloat16
    w = dequantize_w4x16(tensors["qweight"], tensors["wscales"], tensors["wzeros"], out_features, in_features)
    w, bias = undo_adanorm_splits(w, tensors.get("bias"), int(adanorm_splits))
    lin = nn.Linear(int(in_features), int(out_features), bias=bias is not None, dtype=compute, device=device)
    with torch.no_grad():
        lin.weight.copy_(w.to(compute))
        if bias is not None:
            lin.bias.copy_(bias.to(compute))
    lin.requires_grad_(False)
    return lin


class AwqPackedLinear(nn.Module):
    """Packed-resident AWQ W4A16 linear (``models/svdq_awq_packed.py:152-207``): buffers ``weight``
    uint8 [oc, ic/2] (column 2j in the low nibble of byte j), ``wscales`` / ``wzeros`` bf16 [oc, ic/64],
    ``bias`` bf16 [oc] or None; forward = ``cozy_gen_worker::awq_w4a16_mm``."""

    _cozy_awq_packed = True

    def __init__(self, in_features: int, out_features: int, *, bias: bool,
                 compute_dtype: torch.dtype = torch.bfloat16, device=None) -> None:
        super().__init__()
        if compute_dtype != torch.bfloat16:
            raise AwqPackedError(f"AwqPackedLinear computes in bf16, not {compute_dtype}")
        if not awq_packed_supported(out_features, in_features):
            raise AwqPackedError(f"AwqPackedLinear [{out_features}, {in_features}] breaks the packed contract "
                                 f"(out % 16, in % 128)")
        self.compute_dtype = compute_dtype
        self.in_features, self.out_features = int(in_features), int(out_features)
        ng = in_features // GROUP_SIZE
        self.register_buffer("weight", torch.zeros(out_features, in_features // 2, dtype=torch.uint8, device=device))
        self.register_buffer("wscales", torch.zeros(out_features, ng, dtype=compute_dtype, device=device))
        self.register_buffer("wzeros", torch.zeros(out_features, ng, dtype=compute_dtype, device=device))
        if bias:
            self.bias: Optional[nn.Parameter] = nn.Parameter(
                torch.zeros(out_features, dtype=compute_dtype, device=device), requires_grad=False)
        else:
            self.bias = None

    def forward(self, x: Tensor) -> Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.in_features).contiguous()
        y = torch.ops.cozy_gen_worker.awq_w4a16_mm(x2, self.weight, self.wscales, self.wzeros, self.bias)
        return y.reshape(*shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, lane=awq-packed")


def build_awq_packed_linear(tensors: dict[str, Tensor], out_features: int, in_features: int, *,
                            adanorm_splits: int = 1, compute_dtype: Optional[torch.dtype] = None,
                            device=None) -> AwqPackedLinear:
    """Packed-resident module from the on-disk tensors (``models/svdq_awq_packed.py:221-253``): codes
    unpacked and re-packed two per byte, grids un-padded and transposed to [oc, groups], the adaLN row
    interleave and bias offsets undone."""
    compute = compute_dtype or torch.bfloat16
    oc, ic = int(out_features), int(in_features)
    dev = torch.device(device) if device is not None else tensors["qweight"].device
    codes = unpack_w4x16(tensors["qweight"].to(dev), oc, ic)
    scale, zero, gs = scales_and_zeros(tensors["wscales"].to(dev), tensors["wzeros"].to(dev), oc, ic)
    if gs != GROUP_SIZE:
        raise AwqPackedError(f"AWQ group size {gs} != {GROUP_SIZE}: the packed lane serves group {GROUP_SIZE} "
                             f"only (decode_awq_linear serves this layer)")
    bias = tensors.get("bias")
    splits = int(adanorm_splits)
    if splits > 1:
        if oc % splits:
            raise AwqLayoutError(f"out_features {oc} not divisible by adanorm_splits {splits}")
        rows = _undo_interleave_rows(oc, splits, codes.device)
        codes, scale, zero = codes[rows], scale[rows], zero[rows]
        if bias is not None:
            bias = _undo_split_bias(bias.to(codes.device), splits)
    mod = AwqPackedLinear(ic, oc, bias=bias is not None, compute_dtype=compute, device=dev)
    with torch.no_grad():
        mod.weight.copy_((codes[:, 1::2] << 4) | codes[:, 0::2])
        mod.wscales.copy_(scale.to(compute))
        mod.wzeros.copy_(zero.to(compute))
        if bias is not None:
            mod.bias.copy_(bias.reshape(-1).to(compute))
    return mod


def awq_packed_self_check(device="cuda") -> Optional[str]:
    """The reference's packed-lane check (``models/svdq_awq_packed.py:256-285``): the packed module
    against the decoded bf16 Linear at [512, 256] and [768, 256] with 6 adaLN splits, rel-Frobenius
    <= 5e-3; None when it passes, else the failure."""
    for oc, ic, splits in ((512, 256, 1), (768, 256, 6)):
        g = torch.Generator().manual_seed(0)
        w = torch.randn(oc, ic, generator=g) * 0.05
        b = torch.randn(oc, generator=g)
        tensors = encode_awq_linear(w, b, adanorm_splits=splits)
        ref = decode_awq_linear(tensors, oc, ic, adanorm_splits=splits, device=device)
        mod = build_awq_packed_linear(tensors, oc, ic, adanorm_splits=splits, device=device)
        x = torch.randn(3, ic, generator=g).to(device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            got, want = mod(x).float(), ref(x).float()
        rel = ((got - want).norm() / want.norm().clamp(min=1e-9)).item()
        if rel > 5e-3:
            return f"awq packed rel err {rel:.4f} vs decoded Linear at [{oc},{ic}] splits={splits}"
    return None


__all__ = [
    "AwqLayoutError", "AwqPackedError", "AwqPackedLinear", "GROUP_SIZE", "apply_adanorm_splits",
    "awq_packed_self_check", "awq_packed_supported", "build_awq_packed_linear", "decode_awq_linear",
    "dequantize_w4x16", "encode_awq_linear", "is_awq_linear", "num_scale_rows", "pack_w4x16",
    "scales_and_zeros", "undo_adanorm_splits", "unpack_w4x16",
]
