"""W8A8 int8 linear layer and its offline producer.

``Int8ScaledLinear`` is the int8 counterpart of the reference's
``_Fp8ScaledLinear`` (``src/gen_worker/models/w8a8.py:319-388``): buffers
``weight`` [out, in], ``weight_scale`` [out, 1] fp32, ``input_scale`` [1, 1]
fp32 when the checkpoint carries a static activation scale, optional ``bias``,
optional ``lora_a`` / ``lora_b``; ``gemm_mode`` "rowwise" (per-token
activation scales) or "pertensor" (one activation scale per call). forward =
activation quant in that mode (``:363``) -> scaled int8 GEMM with the
activation scale(s), per-channel weight scales and the bias in the epilogue
(``:366-378``) -> optional LoRA addend (``:379-380``).
The quantizer is the reference's int8 formula (``models/svdq_layout.py:261-275``)
with one block per row.
"""

from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn as nn
from torch import Tensor

from . import ops  # noqa: F401  (registers the ops)

_DIM_ALIGN = 16


class W8a8Error(RuntimeError):
    """Typed W8A8 contract failure."""


def quantize_weight_int8(w: Tensor) -> tuple[Tensor, Tensor]:
    """fp weight [N, K] -> (int8 [N, K], fp32 weight_scale [N, 1]): ``scale = max(amax/127, 1e-12)``,
    ``q = clamp(round(w / scale), -127, 127)`` (``models/svdq_layout.py:267-272``, row blocks)."""
    wf = w.detach().float().cpu()
    scale = (wf.abs().amax(dim=-1, keepdim=True) / 127.0).clamp(min=1e-12)
    q = (wf / scale).round().clamp(-127, 127).to(torch.int8)
    return q, scale.float()


GEMM_MODES = ("rowwise", "pertensor")


class Int8ScaledLinear(nn.Module):
    """W8A8 linear on the HIP int8 GEMM: per-token or per-tensor activation scales (dynamic, or the static
    ``input_scale``) x per-channel weight scales."""

    _cozy_w8a8_linear = True

    def __init__(self, in_features: int, out_features: int, *, bias: bool, compute_dtype: Any = torch.bfloat16,
                 bias_dtype: Optional[torch.dtype] = None, device: Any = None, static_input_scale: bool = False,
                 gemm_mode: str = "rowwise") -> None:
        super().__init__()
        if in_features % 64 or out_features % _DIM_ALIGN:
            raise W8a8Error(f"Int8ScaledLinear [{out_features}, {in_features}] breaks the kernel contract "
                            f"(in%64, out%{_DIM_ALIGN})")
        if gemm_mode not in GEMM_MODES:
            raise W8a8Error(f"Int8ScaledLinear: gemm_mode {gemm_mode!r} is not one of {GEMM_MODES}")
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.compute_dtype = compute_dtype
        self.gemm_mode = gemm_mode
        dev = torch.device(device) if device is not None else torch.device("meta")
        self.register_buffer("weight", torch.empty(out_features, in_features, dtype=torch.int8, device=dev))
        self.register_buffer("weight_scale", torch.empty(out_features, 1, dtype=torch.float32, device=dev))
        # a static activation scale is a state-dict entry of the checkpoints that carry one; dynamic layers
        # have no such key
        self.input_scale: Optional[Tensor]
        if static_input_scale:
            self.register_buffer("input_scale", torch.empty(1, 1, dtype=torch.float32, device=dev))
        else:
            self.input_scale = None
        if bias:
            self.bias: Optional[nn.Parameter] = nn.Parameter(
                torch.empty(out_features, dtype=bias_dtype or compute_dtype, device=dev), requires_grad=False)
        else:
            self.bias = None
        self.register_buffer("lora_a", None, persistent=False)
        self.register_buffer("lora_b", None, persistent=False)
        # the operands bound for eager calls (ops.BoundLinearW8a8), rebuilt when any of them changes
        self._bound: Optional[ops.BoundLinearW8a8] = None

    def _lora_addend(self, x2: Tensor) -> Tensor:
        return (x2 @ self.lora_a.t()) @ self.lora_b.t()

    def forward(self, x: Tensor) -> Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype != torch.bfloat16:
            raise W8a8Error(f"Int8ScaledLinear expects bf16 activations, got {x2.dtype}")
        x2 = x2.contiguous()
        y = self._eager(x2) if ops.eager_call_ok(x2) else None
        if y is None:
            xq, sa = torch.ops.cozy_gen_worker.w8a8_quant(x2, self.gemm_mode == "pertensor", self.input_scale)
            y = torch.ops.cozy_gen_worker.w8a8_scaled_mm(xq, self.weight, sa, self.weight_scale, self.bias,
                                                         self.compute_dtype)
        if self.lora_a is not None:
            y = y + self._lora_addend(x2)
        return y.reshape(*shape[:-1], self.out_features)

    def _eager(self, x2: Tensor) -> Optional[Tensor]:
        """The quant and the GEMM through the bound call (the ops' entry points and arguments, no dispatcher);
        None when ``x2`` does not fit it. The binding holds the operand tensors it was made from and is remade
        when an operand attribute names another tensor or storage, or the mode or output dtype changes."""
        ts = (self.weight, self.weight_scale, self.bias, self.input_scale)
        key = (tuple(None if t is None else (id(t), t.data_ptr()) for t in ts), self.gemm_mode, self.compute_dtype)
        b = self._bound
        if b is None or b.key != key:
            b = self._bound = ops.BoundLinearW8a8(
                key=key, held=ts, weight=self.weight, weight_scale=self.weight_scale, bias=self.bias,
                static=self.input_scale, pertensor=self.gemm_mode == "pertensor", out_dtype=self.compute_dtype)
        return b(x2)

    def _apply(self, fn: Any, recurse: bool = True) -> "Int8ScaledLinear":
        """Module moves and casts drop the eager binding (it is remade from the moved buffers)."""
        super()._apply(fn, recurse)
        self._bound = None
        return self

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, gemm_mode={self.gemm_mode}, "
                f"static_input_scale={self.input_scale is not None}")


def build_int8_linear(*, qweight: Tensor, weight_scale: Tensor, bias: Optional[Tensor],
                      compute_dtype: Any = torch.bfloat16, device: Any = "cuda",
                      input_scale: Optional[Tensor] = None, gemm_mode: str = "rowwise") -> Int8ScaledLinear:
    n, k = int(qweight.shape[0]), int(qweight.shape[1])
    mod = Int8ScaledLinear(k, n, bias=bias is not None, compute_dtype=compute_dtype,
                           bias_dtype=bias.dtype if bias is not None else None, device=device,
                           static_input_scale=input_scale is not None, gemm_mode=gemm_mode)
    with torch.no_grad():
        mod.weight.copy_(qweight.to(torch.int8))
        mod.weight_scale.copy_(weight_scale.float().reshape(n, 1))
        if input_scale is not None:
            if input_scale.numel() != 1:
                raise W8a8Error(f"input_scale has {input_scale.numel()} values; a static activation scale is "
                                f"one scalar")
            mod.input_scale.copy_(input_scale.float().reshape(1, 1))
        if bias is not None:
            mod.bias.copy_(bias.reshape(-1))
    return mod


def quantize_linear_w8a8(linear: nn.Linear, *, compute_dtype: Any = torch.bfloat16,
                         device: Any = "cuda") -> Int8ScaledLinear:
    """Producer (``quantize_tree_w8a8``, ``models/w8a8.py:738-792``, int8 form)."""
    q, s = quantize_weight_int8(linear.weight)
    b = linear.bias.detach().to(compute_dtype) if linear.bias is not None else None
    return build_int8_linear(qweight=q, weight_scale=s, bias=b, compute_dtype=compute_dtype, device=device)


def dequantized_linear(*, qweight: Tensor, weight_scale: Tensor, bias: Optional[Tensor],
                       compute_dtype: Any = torch.bfloat16, device: Any = "cuda") -> nn.Linear:
    """The dequant lane's module: one ``nn.Linear`` holding ``qweight * weight_scale`` in ``compute_dtype``
    (``models/w8a8.py:484-488``: the weight's memory saving is given up, its numbers are kept)."""
    n, k = int(qweight.shape[0]), int(qweight.shape[1])
    s = weight_scale.detach().float().reshape(-1)
    if s.numel() not in (1, n):
        raise W8a8Error(f"weight_scale has {s.numel()} values for {n} output channels")
    w = qweight.detach().float() * s.reshape(-1, 1).to(qweight.device)
    lin = nn.Linear(k, n, bias=bias is not None, device="meta")
    lin.weight = nn.Parameter(w.to(device=device, dtype=compute_dtype), requires_grad=False)
    if bias is not None:
        lin.bias = nn.Parameter(bias.detach().reshape(-1).to(device=device, dtype=compute_dtype),
                                requires_grad=False)
    return lin


def serving_w8a8_linear(*, qweight: Tensor, weight_scale: Tensor, bias: Optional[Tensor],
                        compute_dtype: Any = torch.bfloat16, device: Any = "cuda",
                        input_scale: Optional[Tensor] = None, mode: Optional[str] = None) -> nn.Module:
    """The module to serve for one W8A8 layer: an ``Int8ScaledLinear`` in ``mode`` ("rowwise" or
    "pertensor"; default: the branch this process qualified, ``qualify.w8a8_gemm_mode``, chosen once), or in
    the dequant lane (``mode="dequant"``, or no branch qualified) the dequantized ``nn.Linear``: the
    reference's loader rule (``models/w8a8.py:462-466``, ``:478-488``)."""
    from .qualify import resolve_w8a8_mode

    mode = resolve_w8a8_mode(mode)
    if mode == "dequant":
        return dequantized_linear(qweight=qweight, weight_scale=weight_scale, bias=bias,
                                  compute_dtype=compute_dtype, device=device)
    return build_int8_linear(qweight=qweight, weight_scale=weight_scale, bias=bias, compute_dtype=compute_dtype,
                             device=device, input_scale=input_scale, gemm_mode=mode)


__all__ = ["GEMM_MODES", "Int8ScaledLinear", "W8a8Error", "build_int8_linear", "dequantized_linear",
           "quantize_linear_w8a8", "quantize_weight_int8", "serving_w8a8_linear"]
