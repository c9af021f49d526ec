"""nvfp4 compatibility lane: the reference's modelopt nvfp4 W4A4 linears on MI355X.

The reference's standalone W4A4 lane (``src/gen_worker/models/w4a4.py``)
stores each linear as ``weight`` uint8 [out, in/2] (e2m1 codes, element 2j in
the low nibble), ``weight_scale`` e4m3 per block of 16 inputs in the cuBLAS
128 x 4 blocked order (``to_blocked_scales``, ``models/nvfp4_quant.py:72-84``),
``weight_scale_2`` fp32, and optional ``input_scale`` / ``pre_quant_scale``
/ ``bias`` (``_W4A4Linear``, ``models/w4a4.py:292-359``). Its forward
quantizes the activations to nvfp4 (``quantize_activation``, bit-identical to
the torch chain ``:92-103``) and runs ``torch._scaled_mm`` on fp4 operands
(``models/w4a4.py:173-180``), a Blackwell instruction.

CDNA4's block-scaled MFMA takes E8M0 scales per 32 elements, not e4m3 per 16,
and code * scale has up to 6 significant bits, which no MX element format
holds but bf16 does. So this lane keeps the reference's numerics with:

* ``cozy_gen_worker::nvfp4_quant_act`` (HIP): the activation codes and scales,
  bit-identical to the reference chain, and in the same pass the exact bf16
  values code * scale (``nvfp4_quant_act_dyn``: with the dynamic second-level
  scale max|x| / (6 * 448) computed on the device, one partial-max pass before);
* the weight decoded once to the exact bf16 values code * scale
  (``cozy_gen_worker::nvfp4_dequant``, HIP) and kept resident;
* one plain bf16 GEMM (``F.linear``: hipBLASLt, fp32 accumulation, bf16 out),
  the same sum of exact products that ``_scaled_mm`` forms, then
  ``* bf16(s2 * weight_scale_2)`` and ``+ bias`` rounded to bf16 step by step,
  as the reference's forward does (``cozy_gen_worker::nvfp4_scale_bias``, HIP,
  one pass).

It is a compatibility lane (checkpoints in the reference's nvfp4 format run
with the reference's activation quantization); its GEMM runs at the bf16 rate.
``quantize_nvfp4_tensor`` is the reference's offline weight quantizer
(``models/w4a4.py:140-154``), used to produce such checkpoints.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import ops  # noqa: F401  (registers cozy_gen_worker::nvfp4_*)

BLOCK = 16
E2M1_MAX = 6.0
FP8_MAX = 448.0
SCALE_MIN = 2.0 ** -9


class Nvfp4Error(ValueError):
    """The nvfp4 tensors do not match the contract."""


def blocked_scale_index(rows: int, kblocks: int, device=None) -> Tensor:
    """int64 [rows, kblocks]: the position of scale (r, c) in the blocked layout."""
    ncb = (kblocks + 3) // 4
    r = torch.arange(rows, device=device).unsqueeze(1)
    c = torch.arange(kblocks, device=device).unsqueeze(0)
    return ((r // 128) * ncb + c // 4) * 512 + (r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4


def to_blocked_scales(scales: Tensor) -> Tensor:
    """Flat per-block scales [rows, kblocks] (e4m3) -> the blocked layout (zero padded), e4m3."""
    rows, kb = (int(d) for d in scales.shape)
    raw = scales.view(torch.uint8) if scales.dtype == torch.float8_e4m3fn else scales
    out = torch.zeros(ops.nvfp4_blocked_scale_numel(rows, kb), dtype=torch.uint8, device=scales.device)
    out[blocked_scale_index(rows, kb, scales.device).reshape(-1)] = raw.reshape(-1)
    return out.view(torch.float8_e4m3fn)


def from_blocked_scales(blocked: Tensor, rows: int, kblocks: int) -> Tensor:
    """The blocked layout -> flat [rows, kblocks] (e4m3)."""
    raw = blocked.view(torch.uint8) if blocked.dtype == torch.float8_e4m3fn else blocked
    flat = raw.reshape(-1)[blocked_scale_index(rows, kblocks, blocked.device)]
    return flat.view(torch.float8_e4m3fn)


_E2M1_BOUNDS = (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0)


def _cast_e2m1(q: Tensor) -> Tensor:
    a = q.abs()
    code = torch.zeros(q.shape, dtype=torch.uint8, device=q.device)
    for b in _E2M1_BOUNDS:
        code += (a > b).to(torch.uint8)
    code += ((a == 0.75) | (a == 1.75) | (a == 2.5)).to(torch.uint8)
    return code + (q < 0).to(torch.uint8) * 8


def quantize_nvfp4_tensor(w: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """The reference's offline weight quantizer (``models/w4a4.py:140-154``): a 2-D float tensor -> (packed
    uint8 [out, in/2], flat e4m3 scales [out, in/16], fp32 weight_scale_2)."""
    wf = w.float()
    n, k = (int(d) for d in wf.shape)
    if k % BLOCK:
        raise Nvfp4Error(f"in_features {k} is not a multiple of {BLOCK}")
    ws2 = (wf.abs().amax() / (E2M1_MAX * FP8_MAX)).clamp(min=1e-12)
    blocks = wf.reshape(n, k // BLOCK, BLOCK)
    bs = blocks.abs().amax(dim=-1) / (E2M1_MAX * ws2)
    bs[bs == 0] = 1.0
    bs8 = bs.clamp(min=SCALE_MIN, max=FP8_MAX).to(torch.float8_e4m3fn)
    q = blocks / (bs8.float().unsqueeze(-1) * ws2)
    codes = _cast_e2m1(q.reshape(n, k))
    return ((codes[:, 1::2] << 4) | codes[:, 0::2]).contiguous(), bs8, ws2


def dynamic_input_scale(x2: Tensor) -> Tensor:
    """The forward's per-tensor second-level scale without a static input_scale (``models/w4a4.py:342-343``):
    max |x| / (6 * 448), at least 1e-12; max |x| taken as max(-min, max) of one aminmax pass (exact)."""
    lo, hi = torch.aminmax(x2)
    return (torch.maximum(-lo, hi).float() / (E2M1_MAX * FP8_MAX)).clamp(min=1e-12)


class Nvfp4Linear(nn.Module):
    """``_W4A4Linear`` (``models/w4a4.py:292-359``) on the MI355X lane: the activation codes of the reference,
    the product on exact bf16 values. Buffers: ``weight_dq`` bf16 [out, in] (code * weight_scale, exact),
    ``weight_scale_2`` fp32 [1, 1], optional ``input_scale`` fp32 [1, 1] and ``pre_quant_scale`` [in];
    ``bias``. bf16 compute only."""

    _cozy_w4a4_linear = True

    def __init__(self, weight_dq: Tensor, weight_scale_2: Tensor, bias: Optional[Tensor],
                 input_scale: Optional[Tensor], pre_quant_scale: Optional[Tensor]) -> None:
        super().__init__()
        self.out_features, self.in_features = (int(d) for d in weight_dq.shape)
        self.compute_dtype = torch.bfloat16
        self.register_buffer("weight_dq", weight_dq)
        self.register_buffer("weight_scale_2", weight_scale_2.float().reshape(1, 1))
        self.register_buffer("input_scale", None if input_scale is None else input_scale.float().reshape(1, 1))
        self.register_buffer("pre_quant_scale",
                             None if pre_quant_scale is None else pre_quant_scale.to(torch.bfloat16))
        self.bias = None if bias is None else nn.Parameter(bias.to(torch.bfloat16), requires_grad=False)

    def forward(self, x: Tensor) -> Tensor:
        if x.dtype != torch.bfloat16:
            raise Nvfp4Error(f"Nvfp4Linear computes in bf16, got {x.dtype}")
        shape = x.shape
        x2 = x.reshape(-1, self.in_features)
        if self.pre_quant_scale is not None:
            x2 = x2 * self.pre_quant_scale
        if self.input_scale is not None:
            s2 = self.input_scale.reshape(())
            _, _, xdq = torch.ops.cozy_gen_worker.nvfp4_quant_act(x2.contiguous(), s2, False, True)
        else:   # s2 = max|x| / (6 * 448) computed on the device, in the quantizer's launch
            _, _, xdq, s2 = torch.ops.cozy_gen_worker.nvfp4_quant_act_dyn(x2.contiguous(), False, True)
        y = F.linear(xdq, self.weight_dq)
        torch.ops.cozy_gen_worker.nvfp4_scale_bias(y, s2, self.weight_scale_2.reshape(()), self.bias)
        return y.reshape(*shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, static_input_scale={self.input_scale is not None}, "
                f"pre_quant_scale={self.pre_quant_scale is not None}")


def build_nvfp4_linear(weight: Tensor, weight_scale: Tensor, weight_scale_2: Tensor, *,
                       bias: Optional[Tensor] = None, input_scale: Optional[Tensor] = None,
                       pre_quant_scale: Optional[Tensor] = None, device="cuda") -> Nvfp4Linear:
    """An ``Nvfp4Linear`` from the contract tensors (``weight_scale`` in the blocked layout the reference's
    module stores, ``models/w4a4.py:317-320``, or flat [out, in/16]); the weight is decoded once on the GPU."""
    if weight.dtype != torch.uint8 or weight.dim() != 2:
        raise Nvfp4Error(f"weight must be uint8 [out, in/2], got {weight.dtype} {tuple(weight.shape)}")
    n, k = int(weight.shape[0]), 2 * int(weight.shape[1])
    if k % BLOCK:
        raise Nvfp4Error(f"in_features {k} is not a multiple of {BLOCK}")
    kb = k // BLOCK
    sc = weight_scale.view(torch.uint8) if weight_scale.dtype == torch.float8_e4m3fn else weight_scale
    if sc.dtype != torch.uint8:
        raise Nvfp4Error(f"weight_scale must be float8_e4m3fn (or its bytes), got {weight_scale.dtype}")
    if sc.numel() == n * kb and tuple(sc.shape) == (n, kb):
        blocked = False
    elif sc.numel() == ops.nvfp4_blocked_scale_numel(n, kb):
        blocked = True
    else:
        raise Nvfp4Error(f"weight_scale has {sc.numel()} entries for [{n}, {kb}] blocks")
    wdq = torch.ops.cozy_gen_worker.nvfp4_dequant(weight.to(device).contiguous(), sc.to(device).contiguous(),
                                                  blocked)
    return Nvfp4Linear(wdq, weight_scale_2.to(device), None if bias is None else bias.to(device),
                       None if input_scale is None else input_scale.to(device),
                       None if pre_quant_scale is None else pre_quant_scale.to(device)).to(device)
