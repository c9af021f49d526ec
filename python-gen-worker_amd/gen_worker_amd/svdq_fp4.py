"""nunchaku SVDQuant fp4 checkpoints: the packaging the reference serves, decoded and run on MI355X.

The reference's svdq lane serves nunchaku's "v1 single-file" fp4 packaging (``models/svdq_layout.py``,
``models/svdq_native.py:94-163``). Per linear the file stores:

* ``qweight`` int8 [out, in/2]: e2m1 codes in deepcompressor's mma fragment interleave (the same
  interleave as the int4 packaging, ``svdq_checkpoint.unpack_qweight``);
* ``wscales`` e4m3 [in/16, out]: one scale per 16 inputs in ``pack_micro_scale``'s order
  (``svdq_layout.py:114-125``): per 128 output rows and 4 consecutive blocks, rows in the order
  (8-row lane c, 4-row b, 4-row a) with row = 32 a + 8 b + c, the 4 blocks innermost;
* ``wcscales`` [out] (``pack_scale`` vector) or ``wtscale`` (scalar): the second-level weight scale;
* ``smooth_factor`` [in], ``bias`` [out] (``pack_scale`` vectors) and the low-rank branch
  ``proj_down`` / ``proj_up`` (16 x 16 packs, or plain int8 / e4m3 with block scales), as in the
  int4 packaging.

The reference's forward (``_SvdqLinear``, ``models/svdq_native.py:140-156``): ``xs = x / smooth``,
``s2 = max|xs| / (6 * 448)``, nvfp4 activation codes, the fp4 GEMM to bf16, ``y * bf16(s2 * ws2)``,
``+ (x @ proj_down) @ proj_up^T``, ``+ bias``. It needs Blackwell fp4 tensor cores; without them the
reference serves the dense fold (``models/svdq_native.py:279``, ``:200-221``), and so does
``svdq_checkpoint.build_module`` here by default. ``SvdqFp4Linear`` is the blockwise numerics on MI355X:
the activation codes and scales of the nvfp4 lane's quantizer (bit-identical to the reference's chain),
the product on the exact bf16 values code * scale (one bf16 GEMM; CDNA4's block-scaled MFMA takes E8M0
scales per 32, not e4m3 per 16), and the reference's bf16 rounding steps after it.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import ops  # noqa: F401  (registers cozy_gen_worker::nvfp4_*)
from .svdq_checkpoint import (SvdqLayoutError, _decode_lowrank, unpack_qweight, unpack_vector)

BLOCK = 16                 # inputs per e4m3 micro-scale
E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
_WARP_N = 128


def unpack_micro_scales(wscales: Tensor, out_features: int, in_features: int) -> Tensor:
    """``pack_micro_scale`` grid [in/16, out] (e4m3) -> row-major [out, in/16] (e4m3)."""
    n, nb = int(out_features), int(in_features) // BLOCK
    if n % _WARP_N or int(in_features) % BLOCK or nb % 4:
        raise SvdqLayoutError(f"svdq fp4 wscales for [{n}, {in_features}] break the micro-scale pack "
                              f"(out % {_WARP_N}, (in / {BLOCK}) % 4)")
    if tuple(wscales.shape) != (nb, n):
        raise SvdqLayoutError(f"svdq fp4 wscales shape {tuple(wscales.shape)} != {(nb, n)}")
    raw = wscales.contiguous().view(torch.uint8)
    # stored (t, block quad q, row c, row b, row a, block j); row = 128 t + 32 a + 8 b + c, block = 4 q + j
    s = raw.reshape(n // _WARP_N, nb // 4, 8, 4, 4, 4).permute(0, 4, 3, 2, 1, 5)
    return s.reshape(n, nb).contiguous().view(torch.float8_e4m3fn)


def pack_micro_scales(scales: Tensor) -> Tensor:
    """Row-major [out, in/16] (e4m3) -> the ``pack_micro_scale`` grid [in/16, out] (for synthetic files)."""
    n, nb = int(scales.shape[0]), int(scales.shape[1])
    if n % _WARP_N or nb % 4:
        raise SvdqLayoutError(f"svdq fp4 scales [{n}, {nb}] break the micro-scale pack")
    raw = scales.contiguous().view(torch.uint8)
    s = raw.reshape(n // _WARP_N, 4, 4, 8, nb // 4, 4).permute(0, 4, 3, 2, 1, 5)
    return s.contiguous().reshape(nb, n).view(torch.float8_e4m3fn)


@dataclass(frozen=True)
class DecodedFp4Linear:
    """One fp4 svdq linear in the logical domain: ``codes`` uint8 [out, in] e2m1 nibbles (bit 3 the sign),
    ``scales`` e4m3 [out, in/16], ``second`` fp32 [out] (per channel) or [1], ``proj_down`` [in, rank] and
    ``proj_up`` [out, rank] bf16, ``smooth_factor`` [in] and ``bias`` [out] bf16 (or None). Field names match
    ``svdq_checkpoint.DecodedInt4Linear``, so the fused-projection split applies to both."""

    out_features: int
    in_features: int
    codes: Tensor
    scales: Tensor
    second: Tensor
    rank: int = 0
    proj_down: Optional[Tensor] = None
    proj_up: Optional[Tensor] = None
    smooth_factor: Optional[Tensor] = None
    bias: Optional[Tensor] = None


def is_fp4_svdq_linear(tensors: dict) -> bool:
    """The fp4 packaging stores e4m3 micro-scales (the int4 one: 16-bit group-64 scales)."""
    ws = tensors.get("wscales")
    return "qweight" in tensors and ws is not None and ws.dtype == torch.float8_e4m3fn


def decode_fp4_linear(tensors: dict, out_features: int, in_features: int, *,
                      lowrank_quant: Optional[str] = "bf16") -> DecodedFp4Linear:
    """One fp4 svdq linear's stored tensors -> :class:`DecodedFp4Linear` (``decode_linear``,
    ``models/svdq_layout.py:363-438``); ``lowrank_quant`` as ``svdq_checkpoint.decode_int4_linear`` takes it."""
    missing = [k for k in ("qweight", "wscales") if k not in tensors]
    if missing:
        raise SvdqLayoutError(f"not an svdq W4A4 linear (missing {missing})")
    if not is_fp4_svdq_linear(tensors):
        raise SvdqLayoutError(f"wscales of dtype {tensors['wscales'].dtype}: not an fp4 svdq linear (its "
                              f"micro-scales are e4m3)")
    n, k = int(out_features), int(in_features)
    codes = unpack_qweight(tensors["qweight"], n, k)
    scales = unpack_micro_scales(tensors["wscales"], n, k)
    if "wcscales" in tensors:
        if int(tensors["wcscales"].numel()) != n:
            raise SvdqLayoutError(f"wcscales numel {int(tensors['wcscales'].numel())} != out_features {n}")
        second = unpack_vector(tensors["wcscales"].float().reshape(-1), n)
    elif "wtscale" in tensors:
        second = tensors["wtscale"].float().reshape(1)
    else:
        raise SvdqLayoutError("svdq fp4 linear has neither wcscales nor wtscale")
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
    return DecodedFp4Linear(n, k, codes, scales, second.float(), rank, down, up, smooth, bias)


def dequantize_fp4_decoded(dec: DecodedFp4Linear) -> Tensor:
    """fp32 [out, in] = e2m1(code) * scale * second (``dequantize_decoded``, ``models/svdq_layout.py:489-501``:
    code * scale is exact in fp32, the second factor rounds once)."""
    lut = torch.tensor(E2M1_VALUES + tuple(-v for v in E2M1_VALUES), dtype=torch.float32, device=dec.codes.device)
    vals = lut[dec.codes.long()].reshape(dec.out_features, -1, BLOCK)
    w = (vals * dec.scales.float().unsqueeze(-1)).reshape(dec.out_features, dec.in_features)
    return w * (dec.second.float().reshape(-1, 1) if dec.second.numel() > 1 else dec.second.float().reshape(()))


def fp4_shape_supported(out_features: int, in_features: int) -> bool:
    """The reference's fp4 GEMM alignment (``models/svdq_native.py:107-110``: in % 32, out % 16)."""
    return in_features % 32 == 0 and out_features % 16 == 0


class SvdqFp4Linear(nn.Module):
    """``_SvdqLinear`` (``models/svdq_native.py:94-163``) on MI355X, bf16 compute. Buffers: ``weight_dq`` bf16
    [out, in] (code * micro-scale, exact), ``weight_scale_2`` fp32 [1, out] or [1, 1], ``smooth_factor`` [in],
    ``proj_down`` [in, rank], ``proj_up`` [out, rank], ``bias``."""

    _cozy_svdq_linear = True

    def __init__(self, weight_dq: Tensor, weight_scale_2: Tensor, *, smooth: Optional[Tensor],
                 proj_down: Optional[Tensor], proj_up: Optional[Tensor], bias: Optional[Tensor]) -> None:
        super().__init__()
        self.out_features, self.in_features = (int(d) for d in weight_dq.shape)
        if not fp4_shape_supported(self.out_features, self.in_features):
            raise SvdqLayoutError(f"SvdqFp4Linear [{self.out_features}, {self.in_features}] breaks the fp4 GEMM "
                                  f"alignment (in % 32, out % 16)")
        if (proj_down is None) != (proj_up is None):
            raise SvdqLayoutError("SvdqFp4Linear: proj_down and proj_up must both be given or both be None")
        self.compute_dtype = torch.bfloat16
        self.rank = int(proj_down.shape[1]) if proj_down is not None else 0
        self.per_channel_scale = weight_scale_2.numel() > 1
        self.register_buffer("weight_dq", weight_dq.to(torch.bfloat16))
        self.register_buffer("weight_scale_2", weight_scale_2.float().reshape(1, -1))
        self.register_buffer("smooth_factor", None if smooth is None else smooth.to(torch.bfloat16).reshape(-1))
        self.register_buffer("proj_down", None if proj_down is None else proj_down.to(torch.bfloat16).contiguous())
        self.register_buffer("proj_up", None if proj_up is None else proj_up.to(torch.bfloat16).contiguous())
        self.bias = None if bias is None else nn.Parameter(bias.to(torch.bfloat16).reshape(-1), requires_grad=False)

    def forward(self, x: Tensor) -> Tensor:
        if x.dtype != torch.bfloat16:
            raise SvdqLayoutError(f"SvdqFp4Linear computes in bf16, got {x.dtype}")
        shape = x.shape
        x2 = x.reshape(-1, self.in_features).contiguous()
        xs = x2 if self.smooth_factor is None else x2 / self.smooth_factor
        # codes, micro-scales and the exact values code * scale, with s2 = max|xs| / (6 * 448) on the device
        _, _, xdq, s2 = torch.ops.cozy_gen_worker.nvfp4_quant_act_dyn(xs.contiguous(), False, True)
        y = F.linear(xdq, self.weight_dq)
        y = y * (s2 * self.weight_scale_2).to(y.dtype)
        if self.proj_down is not None:
            y = y + F.linear(x2 @ self.proj_down, self.proj_up)
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, rank={self.rank}, "
                f"bias={self.bias is not None}, per_channel_scale={self.per_channel_scale}, "
                f"smooth={self.smooth_factor is not None}")


# "blockwise": SvdqFp4Linear (the reference's fp4 numerics); "dense": one folded bf16 Linear, which the reference
# serves wherever its fp4 GEMM is unavailable (``models/svdq_native.py:279``, ``:399``), so the default here
FP4_MODES = ("blockwise", "dense")


def resolve_fp4_mode(mode: Optional[str] = None) -> str:
    if mode in (None, ""):
        return "dense"
    if mode not in FP4_MODES:
        raise SvdqLayoutError(f"svdq fp4 mode {mode!r}: not one of {', '.join(FP4_MODES)}")
    return mode


def build_fp4_module(dec: DecodedFp4Linear, *, device: Any = "cuda", mode: Optional[str] = None) -> nn.Module:
    """The device module for one decoded fp4 linear (``swap_svdq_linears``, ``models/svdq_native.py:297-316``):
    ``SvdqFp4Linear`` in the blockwise mode when the shape meets the fp4 alignment, else the folded Linear."""
    from .svdq_checkpoint import fold_decoded

    if resolve_fp4_mode(mode) == "blockwise" and fp4_shape_supported(dec.out_features, dec.in_features):
        return build_svdq_fp4_linear(dec, device=device)
    return fold_decoded(dec, device=device)


def build_svdq_fp4_linear(dec: DecodedFp4Linear, *, device: Any = "cuda") -> SvdqFp4Linear:
    """An ``SvdqFp4Linear`` from a decoded linear; the weight's exact bf16 values are decoded on the GPU."""
    packed = ((dec.codes[:, 0::2] & 0xF) | ((dec.codes[:, 1::2] & 0xF) << 4)).contiguous()
    wdq = torch.ops.cozy_gen_worker.nvfp4_dequant(packed.to(device), dec.scales.view(torch.uint8).to(device)
                                                  .contiguous(), False)
    return SvdqFp4Linear(wdq, dec.second.to(device), smooth=None if dec.smooth_factor is None else
                         dec.smooth_factor.to(device),
                         proj_down=dec.proj_down.to(device) if dec.rank else None,
                         proj_up=dec.proj_up.to(device) if dec.rank else None,
                         bias=None if dec.bias is None else dec.bias.to(device))


__all__ = ["BLOCK", "DecodedFp4Linear", "FP4_MODES", "SvdqFp4Linear", "build_fp4_module", "build_svdq_fp4_linear",
           "decode_fp4_linear", "dequantize_fp4_decoded", "fp4_shape_supported", "is_fp4_svdq_linear",
           "pack_micro_scales", "resolve_fp4_mode", "unpack_micro_scales"]
