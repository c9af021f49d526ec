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
* ``decode_awq_tensors``: one validating decoder from the on-disk tensors to
  ``AwqDecoded`` (codes, scale / zero grids, group size, bias), whose
  ``in_original_order`` undoes the adaLN row interleave; every consumer
  starts from it:
* the packed-resident module ``AwqPackedLinear`` (the reference's packed
  module's buffer names, ``models/svdq_awq_packed.py:152-207``: weight uint8
  [oc, ic/2], wscales / wzeros [oc, ic/64]) whose forward is the
  ``cozy_gen_worker::awq_w4a16_mm`` op, built by
  ``AwqPackedLinear.from_decoded`` / ``build_awq_packed_linear``;
* ``decode_awq_linear``: the any-hardware lane (a plain bf16 ``nn.Linear``
  holding the dequantized weight), ``awq_packed_self_check`` (the packed lane
  against it on the device), and ``encode_awq_linear``, the exporter-layout
  producer used to synthesize inputs.

The TinyChat interleave and the adaLN transform are formats fixed by the
checkpoints, so the functions here compute exactly what the reference's
functions of the same names compute, written independently.
"""

from __future__ import annotations

from dataclasses import dataclass
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


def _live_groups(wscales: Tensor, wzeros: Tensor, oc: int, ic: int) -> tuple[int, int]:
    """(groups, group size) of padded [rows, oc] grids: the groups are the leading rows holding any nonzero
    scale (the exporter zero-fills the padding rows), which must divide in_features, and the padded row
    count must be the exporter's for that group size."""
    if wscales.dim() != 2 or int(wscales.shape[1]) != oc:
        raise AwqLayoutError(f"wscales {tuple(wscales.shape)}: expected [rows, {oc}] for {oc} output channels")
    if tuple(wzeros.shape) != tuple(wscales.shape):
        raise AwqLayoutError(f"wzeros {tuple(wzeros.shape)} and wscales {tuple(wscales.shape)} differ in shape")
    nonzero = (wscales != 0).any(dim=1).tolist()
    groups = nonzero.index(False) if False in nonzero else len(nonzero)
    if groups == 0 or any(nonzero[groups:]):
        raise AwqLayoutError("wscales: the rows holding scales are not a leading block followed by zero padding")
    if ic % groups:
        raise AwqLayoutError(f"{groups} scale groups do not divide in_features {ic}")
    gs = ic // groups
    if int(wscales.shape[0]) != num_scale_rows(ic, gs):
        raise AwqLayoutError(f"wscales has {int(wscales.shape[0])} rows; group size {gs} at in_features {ic} "
                             f"pads to {num_scale_rows(ic, gs)}")
    return groups, gs


def scales_and_zeros(wscales: Tensor, wzeros: Tensor, out_features: int,
                     in_features: int) -> tuple[Tensor, Tensor, int]:
    """Padded grids [rows, oc] -> (scale, zero) fp32 [oc, groups] and the group size (the grid layout of
    ``models/svdq_awq.py:49-71``)."""
    groups, gs = _live_groups(wscales, wzeros, int(out_features), int(in_features))
    return (wscales[:groups].float().t().contiguous(), wzeros[:groups].float().t().contiguous(), gs)


@dataclass(frozen=True)
class AwqDecoded:
    """One AWQ W4A16 linear in logical form: codes uint8 [oc, ic] (0..15), scale and zero fp32
    [oc, groups] (w = code * scale + zero), the group size and the bias as stored; rows in the order the
    tensors hold them (``in_original_order`` undoes the exporter's adaLN row interleave)."""

    codes: Tensor
    scale: Tensor
    zero: Tensor
    group_size: int
    bias: Optional[Tensor]

    @property
    def out_features(self) -> int:
        return int(self.codes.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.codes.shape[1])

    def in_original_order(self, splits: int) -> "AwqDecoded":
        """The layer before the exporter's adaLN transform (``models/svdq_awq.py:85-103`` states it): stored
        row j * splits + s is original row s * per + j, and splits 1 and splits - 2 carry +1 in the bias."""
        if splits <= 1:
            return self
        oc = self.out_features
        if oc % splits:
            raise AwqLayoutError(f"out_features {oc} is not a multiple of adanorm_splits {splits}")
        per = oc // splits
        i = torch.arange(oc, device=self.codes.device)
        stored_row = (i % per) * splits + i // per
        bias = None
        if self.bias is not None:
            bias = _unshift_split_bias(self.bias.float().reshape(per, splits).t(), splits).reshape(oc)
        return AwqDecoded(self.codes[stored_row], self.scale[stored_row], self.zero[stored_row], self.group_size,
                          bias)

    def weight(self) -> Tensor:
        """fp32 [oc, ic] = code * scale + zero."""
        oc, ic, gs = self.out_features, self.in_features, self.group_size
        w = self.codes.float().reshape(oc, ic // gs, gs)
        return (w * self.scale.unsqueeze(-1) + self.zero.unsqueeze(-1)).reshape(oc, ic)


def decode_awq_tensors(tensors: dict[str, Tensor], out_features: int, in_features: int) -> AwqDecoded:
    """The on-disk tensors of one AWQ linear (``qweight``, ``wscales``, ``wzeros``, optional ``bias``),
    validated, in logical form."""
    missing = [k for k in ("qweight", "wscales", "wzeros") if k not in tensors]
    if missing:
        raise AwqLayoutError(f"an AWQ W4A16 linear needs qweight, wscales and wzeros; {', '.join(missing)} missing")
    oc, ic = int(out_features), int(in_features)
    codes = unpack_w4x16(tensors["qweight"], oc, ic)
    scale, zero, gs = scales_and_zeros(tensors["wscales"].to(codes.device), tensors["wzeros"].to(codes.device),
                                       oc, ic)
    bias = tensors.get("bias")
    if bias is not None and int(bias.numel()) != oc:
        raise AwqLayoutError(f"bias has {int(bias.numel())} values for {oc} output channels")
    return AwqDecoded(codes, scale, zero, gs, bias.to(codes.device) if bias is not None else None)


def dequantize_w4x16(qweight: Tensor, wscales: Tensor, wzeros: Tensor, out_features: int,
                     in_features: int) -> Tensor:
    """AWQ tensors -> fp32 weight [oc, ic] = code * scale + zero (rows as stored)."""
    return decode_awq_tensors({"qweight": qweight, "wscales": wscales, "wzeros": wzeros}, out_features,
                              in_features).weight()


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


def _unshift_split_bias(by_split: Tensor, splits: int) -> Tensor:
    """[splits, per] bias without the +1 the exporter folds into splits 1 and splits - 2 (one split when
    they coincide)."""
    return by_split - _split_delta(splits, by_split.dtype, by_split.device).reshape(splits, 1)


def undo_adanorm_splits(weight: Tensor, bias: Optional[Tensor], splits: int) -> tuple[Tensor, Optional[Tensor]]:
    """Inverse of :func:`apply_adanorm_splits` on a dense weight (``models/svdq_awq.py:85-103``)."""
    if splits <= 1:
        return weight, bias
    oc = int(weight.shape[0])
    if oc % splits:
        raise AwqLayoutError(f"out_features {oc} is not a multiple of adanorm_splits {splits}")
    per = oc // splits
    w = weight.reshape(per, splits, -1).transpose(0, 1).reshape(oc, -1)
    if bias is None:
        return w, None
    return w, _unshift_split_bias(bias.float().reshape(per, splits).t(), splits).reshape(oc)


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
    """The any-hardware lane (the role of ``models/svdq_awq.py:106-129``): a plain ``nn.Linear`` in
    ``compute_dtype`` (bf16) holding the dequantized weight in the original row order."""
    dec = decode_awq_tensors(tensors, out_features, in_features).in_original_order(int(adanorm_splits))
    dtype = compute_dtype or torch.bfloat16
    lin = nn.Linear(dec.in_features, dec.out_features, bias=dec.bias is not None, dtype=dtype, device=device)
    with torch.no_grad():
        lin.weight.copy_(dec.weight().to(dtype))
        if dec.bias is not None:
            lin.bias.copy_(dec.bias.to(dtype))
    return lin.requires_grad_(False)


def _packed_contract(out_features: int, in_features: int, compute_dtype: torch.dtype) -> Optional[str]:
    """Why a shape / dtype cannot take the packed lane (None when it can)."""
    if compute_dtype != torch.bfloat16:
        return f"the packed AWQ lane computes in bf16, not {compute_dtype}"
    if not awq_packed_supported(out_features, in_features):
        return (f"the packed AWQ lane needs out_features % 16 == 0 and in_features % 128 == 0, got "
                f"[{out_features}, {in_features}]")
    return None


class AwqPackedLinear(nn.Module):
    """AWQ W4A16 linear served from its packed form (the module of ``models/svdq_awq_packed.py:152-207``,
    same buffer names): ``weight`` uint8 [oc, ic/2] (column 2j in the low nibble of byte j), ``wscales`` /
    ``wzeros`` bf16 [oc, ic/64], ``bias`` bf16 [oc] or None; forward = ``cozy_gen_worker::awq_w4a16_mm``."""

    _cozy_awq_packed = True

    def __init__(self, in_features: int, out_features: int, *, bias: bool,
                 compute_dtype: torch.dtype = torch.bfloat16, device=None) -> None:
        super().__init__()
        why = _packed_contract(int(out_features), int(in_features), compute_dtype)
        if why is not None:
            raise AwqPackedError(why)
        self.in_features, self.out_features = int(in_features), int(out_features)
        self.compute_dtype = compute_dtype
        groups = self.in_features // GROUP_SIZE
        empty = lambda *shape, dtype: torch.zeros(*shape, dtype=dtype, device=device)  # noqa: E731
        self.register_buffer("weight", empty(self.out_features, self.in_features // 2, dtype=torch.uint8))
        self.register_buffer("wscales", empty(self.out_features, groups, dtype=compute_dtype))
        self.register_buffer("wzeros", empty(self.out_features, groups, dtype=compute_dtype))
        self.bias: Optional[nn.Parameter] = (
            nn.Parameter(empty(self.out_features, dtype=compute_dtype), requires_grad=False) if bias else None)

    @classmethod
    def from_decoded(cls, dec: AwqDecoded, *, compute_dtype: Optional[torch.dtype] = None,
                     device=None) -> "AwqPackedLinear":
        """The packed module of a decoded layer (rows as they should be served)."""
        if dec.group_size != GROUP_SIZE:
            raise AwqPackedError(f"the packed AWQ lane serves group size {GROUP_SIZE}, this layer has "
                                 f"{dec.group_size} (decode_awq_linear serves it)")
        dev = torch.device(device) if device is not None else dec.codes.device
        mod = cls(dec.in_features, dec.out_features, bias=dec.bias is not None,
                  compute_dtype=compute_dtype or torch.bfloat16, device=dev)
        codes = dec.codes.to(dev)
        with torch.no_grad():
            mod.weight.copy_(codes[:, 0::2] | (codes[:, 1::2] << 4))
            mod.wscales.copy_(dec.scale.to(dev, mod.compute_dtype))
            mod.wzeros.copy_(dec.zero.to(dev, mod.compute_dtype))
            if dec.bias is not None:
                mod.bias.copy_(dec.bias.reshape(-1).to(dev, mod.compute_dtype))
        return mod

    def forward(self, x: Tensor) -> Tensor:
        lead = x.shape[:-1]
        y = torch.ops.cozy_gen_worker.awq_w4a16_mm(x.reshape(-1, self.in_features).contiguous(), self.weight,
                                                   self.wscales, self.wzeros, self.bias)
        return y.reshape(*lead, self.out_features)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, lane=awq-packed")


def build_awq_packed_linear(tensors: dict[str, Tensor], out_features: int, in_features: int, *,
                            adanorm_splits: int = 1, compute_dtype: Optional[torch.dtype] = None,
                            device=None) -> AwqPackedLinear:
    """The packed module from the on-disk tensors (the role of ``models/svdq_awq_packed.py:221-253``):
    decoded, put back in the original row order, re-packed two codes per byte."""
    src = tensors["qweight"].device if "qweight" in tensors else None
    dev = torch.device(device) if device is not None else src
    on_dev = {k: v.to(dev) for k, v in tensors.items()}
    dec = decode_awq_tensors(on_dev, out_features, in_features).in_original_order(int(adanorm_splits))
    return AwqPackedLinear.from_decoded(dec, compute_dtype=compute_dtype, device=dev)


# (out_features, in_features, adaLN splits, activation rows): the GEMV path and the dequantize + GEMM path
# of awq_w4a16_mm, with and without the adaLN row interleave
_SELF_CHECK_CASES = ((256, 384, 1, 1), (384, 256, 6, 1), (384, 256, 6, 24))
SELF_CHECK_REL_TOL = 5e-3   # the reference's bar for its packed lane (models/svdq_awq_packed.py:256-285)


def awq_packed_self_check(device="cuda") -> Optional[str]:
    """The packed lane against the decoded bf16 Linear of the same tensors on the device: None when every
    case is within ``SELF_CHECK_REL_TOL`` (relative Frobenius error), else the first failing case."""
    for oc, ic, splits, rows in _SELF_CHECK_CASES:
        g = torch.Generator().manual_seed(1000 * splits + rows)
        tensors = encode_awq_linear(torch.randn(oc, ic, generator=g) * 0.04,
                                    torch.randn(oc, generator=g) * 0.1, adanorm_splits=splits)
        packed = build_awq_packed_linear(tensors, oc, ic, adanorm_splits=splits, device=device)
        dense = decode_awq_linear(tensors, oc, ic, adanorm_splits=splits, device=device)
        x = torch.randn(rows, ic, generator=g).to(device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            got, want = packed(x).float(), dense(x).float()
        rel = float((got - want).norm() / want.norm().clamp(min=1e-12))
        if not rel <= SELF_CHECK_REL_TOL:
            return (f"packed AWQ [{oc} x {ic}], {splits} adaLN split(s), {rows} row(s): relative error {rel:.2e} "
                    f"against its decoded Linear exceeds {SELF_CHECK_REL_TOL}")
    return None


__all__ = [
    "AwqDecoded", "AwqLayoutError", "AwqPackedError", "AwqPackedLinear", "GROUP_SIZE", "SELF_CHECK_REL_TOL",
    "apply_adanorm_splits", "awq_packed_self_check", "awq_packed_supported", "build_awq_packed_linear",
    "decode_awq_linear", "decode_awq_tensors", "dequantize_w4x16", "encode_awq_linear", "is_awq_linear",
    "num_scale_rows", "pack_w4x16", "scales_and_zeros", "undo_adanorm_splits", "unpack_w4x16",
]
