"""SVDQuant W4A4 (int4, group 64) linear layer and its offline producers.

``SvdqW4A4Linear`` is the int4-g64 counterpart of the reference's fused lane
module ``_SvdqFusedLinear`` (``src/gen_worker/models/svdq_fused.py:471-534``):
same buffer names (``weight``, ``weight_scale``, ``second``,
``smooth_factor``, ``proj_down``, ``proj_up``, ``bias``), same forward
structure (``:516-527``: quantize -> W4A4 GEMM -> low-rank + bias epilogue),
but two launches instead of four: kernel 1 fuses the smoothing, the act-quant
and ``x2 @ proj_down``; kernel 2 fuses the GEMM with the whole epilogue.
On the GPU (the fp6 lane) kernel 1 writes its codes and scales as fp6
operand records and the GEMM runs on gfx950's fp6 MFMA against weights
prepacked into the same records (``weight_fp6``); an ``in_features`` with
``in_features % 128 == 64`` ends in a half stage whose second group holds zero
codes. The general lane (int4 codes, int8-MFMA GEMM) stays available through
its ops.

Buffer formats (the int4 lane's own layout):
  weight        uint8 [out, in/2]   two's-complement int4 codes, low nibble = even k
  weight_scale  fp16  [out, in/64]  one scale per group of 64 along in_features
  second        fp32  [out] or [1]  per-channel / per-tensor output multiplier
  smooth_factor bf16  [in]          divides the activation of the 4-bit branch only
  proj_down     bf16  [in, rank]    low-rank down factor (applied to RAW x)
  proj_up       bf16  [out, rank]   low-rank up factor
  bias          bf16  [out]
"""

from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn as nn
from torch import Tensor

from . import ops

GROUP = 64
_N_ALIGN = 16
SUPPORTED_RANKS = (0, 16, 32, 64, 128)


class SvdqFusedError(RuntimeError):
    """Typed contract failure of the int4 fused lane (``models/svdq_fused.py:34-35``)."""


def fused_shape_supported(out_features: int, in_features: int, rank: int) -> bool:
    """Shape contract of the kernels (reference: ``models/svdq_fused.py:38-41``)."""
    return (in_features % GROUP == 0 and out_features % _N_ALIGN == 0 and rank in SUPPORTED_RANKS)


# ---------------------------------------------------------------------------
# int4 format helpers (torch; offline/CPU or GPU)
# ---------------------------------------------------------------------------

def pack_int4(codes: Tensor) -> Tensor:
    """int codes [..., K] in [-8, 7] -> uint8 [..., K/2], element 2j in the LOW nibble (``pack_e2m1``, ``models/nvfp4_quant.py:54-56``)."""
    c = (codes.to(torch.int16) & 0xF).to(torch.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).contiguous()


def unpack_int4(packed: Tensor) -> Tensor:
    """uint8 [..., K/2] -> int8 codes [..., K]."""
    p = packed.to(torch.int16)
    lo, hi = p & 0xF, (p >> 4) & 0xF
    out = torch.stack((lo, hi), dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)
    out = torch.where(out >= 8, out - 16, out)
    return out.to(torch.int8)


def quantize_weight_int4(w: Tensor) -> tuple[Tensor, Tensor]:
    """fp weight [N, K] -> (packed uint8 [N, K/2], fp16 scales [N, K/64]).

    Offline producer, structured as ``quantize_nvfp4_tensor``
    (``models/w4a4.py:140-154``): per-block absmax, zero blocks get scale 1,
    clamp, cast the scale to its stored dtype, divide by the stored scale,
    round (RNE) and clamp the codes. Single-level: no second scale.
    """
    wf = w.detach().float().cpu()
    n, k = wf.shape
    if k % GROUP:
        raise SvdqFusedError(f"in_features {k} is not a multiple of {GROUP}")
    blocks = wf.reshape(n, k // GROUP, GROUP)
    bs = blocks.abs().amax(dim=-1) / 7.0
    bs[bs == 0] = 1.0
    bs = bs.clamp(min=2.0 ** -24, max=65504.0).to(torch.float16)
    q = (blocks / bs.float().unsqueeze(-1)).round().clamp(-8, 7).to(torch.int8)
    return pack_int4(q.reshape(n, k)), bs


def dequantize_weight_int4(packed: Tensor, scales: Tensor) -> Tensor:
    """(packed, fp16 scales) -> float32 [N, K] (``dequantize_decoded``, ``models/svdq_layout.py:492-504``)."""
    q = unpack_int4(packed).float()
    n, k = q.shape
    return (q.reshape(n, k // GROUP, GROUP) * scales.float().reshape(n, k // GROUP, 1)).reshape(n, k)


def svdquant_decompose(w: Tensor, smooth: Optional[Tensor], rank: int) -> tuple[Tensor, Tensor, Tensor]:
    """SVDQuant split of a dense weight: W = W_res / smooth + up @ down^T.

    The smoothed weight ``W * smooth`` (smoothing migrates activation
    outliers into the weight) is split by an SVD into a rank-``rank``
    component, kept in 16-bit as ``proj_up @ proj_down^T`` on the RAW
    activations (so ``proj_down`` is pre-divided by ``smooth``, as the
    reference notes in ``models/svdq_layout.py:1``), and a residual that is
    quantized to int4. Returns (w_res [N, K] fp32, proj_down [K, r], proj_up [N, r]).
    """
    wf = w.detach().float().cpu()
    sm = smooth.detach().float().cpu().reshape(1, -1) if smooth is not None else None
    ws = wf * sm if sm is not None else wf
    if rank == 0:
        return ws, wf.new_zeros(wf.shape[1], 0), wf.new_zeros(wf.shape[0], 0)
    u, s, vh = torch.linalg.svd(ws, full_matrices=False)
    up = u[:, :rank] * s[:rank]                # [N, r]
    down_s = vh[:rank].t()                      # [K, r] acting on smoothed x
    res = ws - up @ down_s.t()
    down = down_s / sm.reshape(-1, 1) if sm is not None else down_s
    return res, down, up


# ---------------------------------------------------------------------------
# the module
# ---------------------------------------------------------------------------

class SvdqW4A4Linear(nn.Module):
    """int4-g64 SVDQuant linear on the HIP kernels (the fused lane)."""

    _cozy_svdq_linear = True
    _cozy_svdq_fused = True

    def __init__(self, in_features: int, out_features: int, *, rank: int, bias: bool,
                 compute_dtype: Any = torch.bfloat16, per_channel_scale: bool = False,
                 smooth: bool = True, activation: Optional[str] = None,
                 out_dtype: Optional[torch.dtype] = None, device: Any = None) -> None:
        super().__init__()
        if not fused_shape_supported(out_features, in_features, rank):
            raise SvdqFusedError(
                f"SvdqW4A4Linear [{out_features}, {in_features}] r{rank} breaks the kernel contract "
                f"(in%{GROUP}, out%{_N_ALIGN}, rank in {SUPPORTED_RANKS})")
        if compute_dtype != torch.bfloat16:
            raise SvdqFusedError(f"compute_dtype {compute_dtype}: the int4 lane quantizes bf16 activations")
        if activation not in (None, "gelu_tanh"):
            raise SvdqFusedError(f"activation {activation!r} not in (None, 'gelu_tanh')")
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.rank = int(rank)
        self.compute_dtype = compute_dtype
        self.per_channel_scale = bool(per_channel_scale)
        self.activation = activation
        self.out_dtype = out_dtype
        dev = torch.device(device) if device is not None else torch.device("meta")
        self.register_buffer("weight", torch.empty(out_features, in_features // 2, dtype=torch.uint8, device=dev))
        self.register_buffer("weight_scale", torch.empty(out_features, in_features // GROUP,
                                                         dtype=torch.float16, device=dev))
        self.register_buffer("second", torch.ones(out_features if per_channel_scale else 1,
                                                  dtype=torch.float32, device=dev))
        if smooth:
            self.register_buffer("smooth_factor", torch.empty(in_features, dtype=compute_dtype, device=dev))
        else:
            self.smooth_factor = None
        if self.rank:
            self.register_buffer("proj_down", torch.empty(in_features, self.rank, dtype=compute_dtype, device=dev))
            self.register_buffer("proj_up", torch.empty(out_features, self.rank, dtype=compute_dtype, device=dev))
            # proj_down in the act-quant kernels' operand orders (derived by refresh_derived, GPU only):
            # the general lane's and the fp6 lane's
            self.register_buffer("proj_down_op", None, persistent=False)
            self.register_buffer("proj_down_op6", None, persistent=False)
        else:
            self.proj_down = self.proj_up = self.proj_down_op = self.proj_down_op6 = None
        if bias:
            self.bias: Optional[nn.Parameter] = nn.Parameter(
                torch.empty(out_features, dtype=compute_dtype, device=dev), requires_grad=False)
        else:
            self.bias = None
        self.register_buffer("_one", torch.ones((), dtype=torch.float32, device=dev), persistent=False)
        # resident fast-lane operand records (derived from ``weight`` / ``weight_scale`` by refresh_derived)
        self.register_buffer("weight_fp6", None, persistent=False)
        # token counts up to this run the small-M GEMV on ``weight`` itself (set with the fp6 records)
        self._gemv_max_m = 0
        # the fp6 lane's operands bound for eager calls (ops.BoundLinearFp6), rebuilt when any of them changes
        self._bound: Optional[ops.BoundLinearFp6] = None
        # identity and version counter of each buffer the derived ones were computed from (_primary_versions)
        self._derived_from: Optional[tuple] = None

    def _primary_versions(self) -> tuple:
        """(id, version counter) of ``weight``, ``weight_scale`` and ``proj_down``, the buffers the derived ones
        are computed from: an in-place update (``mod.weight.copy_(...)``) bumps the counter and a reassignment
        changes the id, and either makes the next forward rebuild the derived buffers. A tensor made under
        ``torch.inference_mode`` keeps no counter (its in-place updates need an explicit ``refresh_derived``)."""
        out = []
        for t in (self.weight, self.weight_scale, self.proj_down):
            if t is None:
                out.append(None)
                continue
            try:
                out.append((id(t), t._version))
            except RuntimeError:
                out.append((id(t), None))
        return tuple(out)

    def refresh_derived(self) -> None:
        """Recompute the derived buffers from ``weight`` / ``weight_scale`` / ``proj_down`` (GPU only):
        ``proj_down`` in kernel 1's operand order, and the weights as fp6 operand records (``in_features % 128
        == 64`` ends in a half stage of zero codes). The forward calls it by itself when those buffers changed
        since the last call (``_primary_versions``)."""
        fp6 = self.weight.is_cuda and self.in_features % GROUP == 0
        if self.rank:
            on_gpu = self.proj_down.is_cuda
            self.proj_down_op = torch.ops.cozy_gen_worker.svdq_prep_proj_down(self.proj_down) if on_gpu else None
            self.proj_down_op6 = (torch.ops.cozy_gen_worker.svdq_prep_proj_down_fp6(self.proj_down)
                                  if on_gpu and fp6 else None)
        self.weight_fp6 = None
        self._gemv_max_m = 0
        self._bound = None
        if fp6:
            self.weight_fp6 = torch.ops.cozy_gen_worker.svdq_pack_weight_fp6(self.weight, self.weight_scale)
            self._gemv_max_m = ops.gemv_max_m(self.in_features, self.rank)
        self._derived_from = self._primary_versions()

    def _apply(self, fn: Any, recurse: bool = True) -> "SvdqW4A4Linear":
        """Module moves and casts (``.to()``, ``.cuda()``, ``.cpu()``) copy buffers without the 1 KB of readable
        slack the fp6 GEMM needs after its operand records, and ``proj_down``'s operand orders depend only on
        ``proj_down``: the derived buffers are dropped here and rebuilt from the primary ones on the next
        forward."""
        super()._apply(fn, recurse)
        self.weight_fp6 = None
        self._bound = None
        if self.rank:
            self.proj_down_op = None
            self.proj_down_op6 = None
        return self

    def _load_from_state_dict(self, *args: Any, **kwargs: Any) -> None:  # noqa: D401
        super()._load_from_state_dict(*args, **kwargs)
        if self.weight.device.type != "meta":
            self.refresh_derived()

    @property
    def lane(self) -> str:
        """``"fp6"`` (kernel 1 writes fp6 operand records, fp6-MFMA GEMM) or ``"general"`` (int4 codes,
        int8-MFMA GEMM on the logical weights)."""
        return "fp6" if self.weight_fp6 is not None else "general"

    def _ensure_derived(self) -> None:
        fp6 = self.weight.is_cuda and self.in_features % GROUP == 0
        if ((self.rank and (self.proj_down_op is None or (fp6 and self.proj_down_op6 is None)))
                or (self.weight_fp6 is None and fp6) or self._derived_from != self._primary_versions()):
            self.refresh_derived()

    def _input2d(self, x: Tensor) -> Tensor:
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype != torch.bfloat16:
            raise SvdqFusedError(f"SvdqW4A4Linear expects bf16 activations, got {x2.dtype}")
        return x2.contiguous()

    def forward_records(self, q6: Tensor, la: Optional[Tensor], out_dtype: Optional[torch.dtype] = None) -> Tensor:
        """The fp6-lane GEMM on ready input records [ceil(K/128), M, 104] and la [M, rank] (bf16, or fp32);
        returns [M, out_features]."""
        self._ensure_derived()
        if self.weight_fp6 is None:
            raise SvdqFusedError("forward_records needs the fp6 lane (weights on the GPU)")
        return torch.ops.cozy_gen_worker.svdq_w4a4_linear_fp6(
            q6, self.weight_fp6, None, self.second, la if self.rank else None, self.proj_up, self.bias,
            out_dtype or self.out_dtype or torch.bfloat16, self.activation == "gelu_tanh")

    def forward(self, x: Tensor) -> Tensor:
        shape = x.shape
        x2 = self._input2d(x)
        out_dtype = self.out_dtype or torch.bfloat16
        self._ensure_derived()
        gelu = self.activation == "gelu_tanh"
        m = int(x2.shape[0])
        if self.weight_fp6 is not None and ops.eager_call_ok(x2):
            y = self._eager(x2, out_dtype, gelu)
            if y is not None:
                return y.reshape(*shape[:-1], self.out_features)
        if self.weight_fp6 is not None and 0 < m <= self._gemv_max_m:
            # a few tokens (the DiT's modulation linears): the int4 weight streamed once by the GEMV
            y = torch.ops.cozy_gen_worker.svdq_forward_gemv(
                x2, self.smooth_factor, None, self.proj_down_op6 if self.rank else None, self.weight,
                self.weight_scale, self.second, self.proj_up, self.bias, out_dtype, gelu)
            return y.reshape(*shape[:-1], self.out_features)
        if self.weight_fp6 is not None:
            y = torch.ops.cozy_gen_worker.svdq_forward_fp6(
                x2, self.smooth_factor, None, self.proj_down_op6 if self.rank else None, self.weight_fp6, self.second,
                self.proj_up, self.bias, out_dtype, gelu)
            return y.reshape(*shape[:-1], self.out_features)
        if self.rank:
            qa, sa, la = torch.ops.cozy_gen_worker.svdq_quant_lora(x2, self.smooth_factor, None, self.proj_down_op)
        else:
            qa, sa = torch.ops.cozy_gen_worker.svdq_quant(x2, self.smooth_factor, self._one, False)
            la = None
        y = torch.ops.cozy_gen_worker.svdq_w4a4_linear(
            qa, sa, self.weight, self.weight_scale, None, self.second, la, self.proj_up,
            self.bias, out_dtype, gelu)
        return y.reshape(*shape[:-1], self.out_features)

    def _eager(self, x2: Tensor, out_dtype: torch.dtype, gelu: bool) -> Optional[Tensor]:
        """The fp6 lane's forward through the bound call (the ops' entry points and arguments, no dispatcher);
        None when ``x2`` does not fit it. The binding holds the operand tensors it was made from and is remade
        when any operand attribute names another tensor or storage, or the output dtype, activation or GEMV
        bound changes."""
        pdo6 = self.proj_down_op6 if self.rank else None
        up = self.proj_up if self.rank else None
        ts = (self.weight_fp6, self.weight, self.weight_scale, self.smooth_factor, pdo6, self.second, up, self.bias)
        key = (tuple(None if t is None else (id(t), t.data_ptr()) for t in ts), out_dtype, gelu, self._gemv_max_m)
        b = self._bound
        if b is None or b.key != key:
            b = self._bound = ops.BoundLinearFp6(
                key=key, held=ts, k=self.in_features, smooth=self.smooth_factor, proj_down_op6=pdo6, weight=self.weight,
                weight_scale=self.weight_scale, weight_fp6=self.weight_fp6, second=self.second, proj_up=up,
                bias=self.bias, out_dtype=out_dtype, gelu=gelu, gemv_max_m=self._gemv_max_m)
        return b(x2)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, rank={self.rank}, "
                f"bias={self.bias is not None}, per_channel_scale={self.per_channel_scale}, "
                f"smooth={self.smooth_factor is not None}, activation={self.activation}, lane=int4-g64")


def _fusable(producer: SvdqW4A4Linear, consumer: SvdqW4A4Linear, k_offset: int) -> bool:
    producer._ensure_derived()
    consumer._ensure_derived()
    return (producer.lane == "fp6" and consumer.lane == "fp6" and producer.out_features % ops.FP6_STAGE == 0
            and producer.out_dtype in (None, torch.bfloat16) and k_offset % ops.FP6_STAGE == 0
            and k_offset + producer.out_features == consumer.in_features)


def _next_operands(consumer: SvdqW4A4Linear, k0: int, k1: int) -> tuple[Optional[Tensor], Optional[Tensor]]:
    """The consumer's smoothing factors and operand-order proj_down rows for its input columns [k0, k1)."""
    sm = consumer.smooth_factor[k0:k1] if consumer.smooth_factor is not None else None
    pdo = consumer.proj_down_op6[k0:k1] if consumer.rank else None
    return sm, pdo


def svdq_pair_forward(x: Tensor, first: SvdqW4A4Linear, second: SvdqW4A4Linear) -> Tensor:
    """``second(first(x))`` with ``second``'s activation quantization fused into ``first``'s GEMM epilogue
    (config 2: fc1 -> GELU -> fc2). The [M, first.out_features] bf16 intermediate never reaches HBM: the
    epilogue writes ``second``'s fp6 records (bit-identical to quantizing the bf16 output) and per-column-tile
    partials of ``output @ second.proj_down``, summed in a fixed order into ``second``'s bf16 la. Layers that do
    not meet the fused contract (both fp6 lane, first.out_features % 128 == 0, bf16 intermediate) run unfused."""
    if not _fusable(first, second, 0):
        return second(first(x))
    cg = torch.ops.cozy_gen_worker
    shape = x.shape
    x2 = first._input2d(x)
    m = int(x2.shape[0])
    q6, la = cg.svdq_quant_fp6(x2, first.smooth_factor, None, first.proj_down_op6)
    q6n = ops.records_empty(second.in_features // ops.FP6_STAGE, m, x2.device)
    part = (torch.empty(ops.la_partials_next(m, first.out_features), m, second.rank, dtype=torch.float32,
                        device=x2.device) if second.rank else None)
    sm, pdo = _next_operands(second, 0, second.in_features)
    cg.svdq_w4a4_linear_fp6_next(q6, first.weight_fp6, None, first.second, la if first.rank else None,
                                 first.proj_up, first.bias, first.activation == "gelu_tanh", sm, pdo, q6n, part, 0,
                                 False)
    y = second.forward_records(q6n, cg.svdq_la_reduce(part) if part is not None else None)
    return y.reshape(*shape[:-1], second.out_features)


def svdq_concat_forward(consumer: SvdqW4A4Linear, x_a: Tensor, producer: SvdqW4A4Linear, x_b: Tensor) -> Tensor:
    """``consumer(cat([x_a, producer(x_b)], -1))`` (Flux's single-block proj_out over [attention, MLP]) without
    the concatenation: kernel 1 writes the first x_a.shape[-1] / 128 stages of ``consumer``'s input records
    from ``x_a``, ``producer``'s fused epilogue writes the rest, and both store their partials of the input @
    proj_down into one slot buffer, summed in a fixed order into ``consumer``'s la. Falls back to the unfused
    composition outside the fused contract (x_a's width a multiple of 128, both fp6 lane)."""
    ka = int(x_a.shape[-1])
    if not _fusable(producer, consumer, ka):
        return consumer(torch.cat((x_a, producer(x_b)), dim=-1))
    st = SvdqConcat(consumer, producer, x_b, ka)
    st.produce()
    return st.finish(x_a)


class SvdqConcat:
    """``svdq_concat_forward`` in two halves, so a caller can run the producer's half (``produce``: its input
    quantization and its GEMM, whose epilogue writes the consumer's records and partial slots past ``ka``) on
    another stream while x_a is still being computed; ``finish(x_a)`` writes x_a's records and slots (kernel 1),
    reduces the slots and runs the consumer. The two halves write disjoint records and slots, so their order
    does not change a bit. The buffers are allocated on the stream that constructs this."""

    def __init__(self, consumer: SvdqW4A4Linear, producer: SvdqW4A4Linear, x_b: Tensor, ka: int) -> None:
        if not _fusable(producer, consumer, ka):
            raise SvdqFusedError("SvdqConcat: outside the fused contract (x_a's width a multiple of 128, fp6 lane)")
        self.consumer, self.producer, self.ka = consumer, producer, ka
        self.xb2 = producer._input2d(x_b)
        m = self.m = int(self.xb2.shape[0])
        self.q6n = ops.records_empty(consumer.in_features // ops.FP6_STAGE, m, self.xb2.device)
        self.part, self.pa = None, 0
        if consumer.rank:
            self.pa = ops.la_partials_quant(m, ka, consumer.rank)
            pb = ops.la_partials_next(m, producer.out_features)
            self.part = torch.empty(self.pa + pb, m, consumer.rank, dtype=torch.float32, device=self.xb2.device)

    def produce(self) -> None:
        cg = torch.ops.cozy_gen_worker
        consumer, producer, ka = self.consumer, self.producer, self.ka
        q6, la = cg.svdq_quant_fp6(self.xb2, producer.smooth_factor, None, producer.proj_down_op6)
        sm_b, pdo_b = _next_operands(consumer, ka, consumer.in_features)
        cg.svdq_w4a4_linear_fp6_next(q6, producer.weight_fp6, None, producer.second,
                                     la if producer.rank else None, producer.proj_up, producer.bias,
                                     producer.activation == "gelu_tanh", sm_b, pdo_b, self.q6n,
                                     self.part[self.pa:] if self.part is not None else None, ka // ops.FP6_STAGE,
                                     False)

    def finish(self, x_a: Tensor, before_reduce=None) -> Tensor:
        """``before_reduce`` (if given) runs after x_a's records are written and before the slots are summed:
        the point where a caller joins the stream that ran ``produce``."""
        cg = torch.ops.cozy_gen_worker
        consumer, ka = self.consumer, self.ka
        shape = x_a.shape
        xa2 = x_a.reshape(-1, ka)
        if xa2.dtype != torch.bfloat16:
            raise SvdqFusedError(f"svdq_concat_forward expects bf16 activations, got {xa2.dtype}")
        xa2 = xa2.contiguous()
        if int(xa2.shape[0]) != self.m:
            raise SvdqFusedError(f"svdq_concat_forward: {int(xa2.shape[0])} rows in x_a, {self.m} in x_b")
        sm_a, pdo_a = _next_operands(consumer, 0, ka)
        cg.svdq_quant_fp6_into(xa2, sm_a, pdo_a, self.q6n, self.part)
        if before_reduce is not None:
            before_reduce()
        y = consumer.forward_records(self.q6n, cg.svdq_la_reduce(self.part) if self.part is not None else None)
        return y.reshape(*shape[:-1], consumer.out_features)


def build_svdq_w4a4_linear(*, qweight: Tensor, wscales: Tensor, smooth: Optional[Tensor],
                           proj_down: Optional[Tensor], proj_up: Optional[Tensor], bias: Optional[Tensor],
                           second: Optional[Tensor] = None, activation: Optional[str] = None,
                           out_dtype: Optional[torch.dtype] = None, device: Any = "cuda") -> SvdqW4A4Linear:
    """A device-resident module from logical int4 buffers (``build_svdq_fused_linear``, ``models/svdq_fused.py:544-573``)."""
    n, kh = int(qweight.shape[0]), int(qweight.shape[1])
    rank = 0 if proj_down is None else int(proj_down.shape[1])
    per_channel = second is not None and second.numel() > 1
    mod = SvdqW4A4Linear(2 * kh, n, rank=rank, bias=bias is not None, per_channel_scale=per_channel,
                         smooth=smooth is not None, activation=activation, out_dtype=out_dtype, device=device)
    with torch.no_grad():
        mod.weight.copy_(qweight.to(torch.uint8))
        mod.weight_scale.copy_(wscales.to(torch.float16))
        if second is not None:
            mod.second.copy_(second.float().reshape(-1))
        if smooth is not None:
            mod.smooth_factor.copy_(smooth.to(torch.bfloat16).reshape(-1))
        if rank:
            mod.proj_down.copy_(proj_down.to(torch.bfloat16))
            mod.proj_up.copy_(proj_up.to(torch.bfloat16))
        if bias is not None:
            mod.bias.copy_(bias.to(torch.bfloat16).reshape(-1))
    mod.refresh_derived()
    return mod


def quantize_linear_w4a4(linear: nn.Linear, *, rank: int, smooth: Optional[Tensor] = None,
                         activation: Optional[str] = None, device: Any = "cuda") -> SvdqW4A4Linear:
    """Producer: dense ``nn.Linear`` -> SVDQuant int4 module (smoothing, SVD low-rank, int4 residual)."""
    res, down, up = svdquant_decompose(linear.weight, smooth, rank)
    qw, ws = quantize_weight_int4(res)
    return build_svdq_w4a4_linear(qweight=qw, wscales=ws, smooth=smooth, proj_down=down if rank else None,
                                  proj_up=up if rank else None,
                                  bias=linear.bias.detach() if linear.bias is not None else None,
                                  activation=activation, device=device)


def fold_to_dense(mod: SvdqW4A4Linear, *, compute_dtype: Any = torch.bfloat16) -> nn.Linear:
    """The any-hardware fallback lane: ONE dense ``nn.Linear`` equal to the whole int4 linear
    (``fold_to_dense``, ``models/svdq_native.py:200-221``): ``W_eff = deq(W)*second / smooth + up @ down^T``.
    Activation quantization is not part of this lane."""
    w = dequantize_weight_int4(mod.weight.cpu(), mod.weight_scale.cpu())
    w = w * mod.second.float().cpu().reshape(-1, 1)
    if mod.smooth_factor is not None:
        w = w / mod.smooth_factor.float().cpu().reshape(1, -1)
    if mod.rank:
        w = w + mod.proj_up.float().cpu() @ mod.proj_down.float().cpu().t()
    lin = nn.Linear(mod.in_features, mod.out_features, bias=mod.bias is not None, dtype=compute_dtype)
    with torch.no_grad():
        lin.weight.copy_(w.to(compute_dtype))
        if mod.bias is not None:
            lin.bias.copy_(mod.bias.detach().cpu().to(compute_dtype))
    lin.weight.requires_grad_(False)
    if lin.bias is not None:
        lin.bias.requires_grad_(False)
    return lin


def w4a4_int_ops(m: int, n: int, k: int) -> int:
    """Algorithmic integer ops of the GEMM, 2*M*N*K."""
    return 2 * m * n * k


def act_quant_bytes(m: int, k: int, rank: int, smooth: bool = True, fp6: bool = False) -> int:
    """Minimal HBM bytes of kernel 1: x, smooth, L1, codes + scales (int4 + fp16, or the fp6 operand
    records: 104 bytes per 128 columns), la (bf16, or fp32 in the fp6 lane)."""
    out = m * (k // ops.FP6_STAGE) * 104 if fp6 else m * k // 2 + m * (k // GROUP) * 2
    return m * k * 2 + (k * 2 if smooth else 0) + k * rank * 2 + out + m * rank * (4 if fp6 else 2)


__all__ = [
    "SvdqFusedError", "SvdqW4A4Linear", "build_svdq_w4a4_linear", "dequantize_weight_int4",
    "fold_to_dense", "fused_shape_supported", "pack_int4", "quantize_linear_w4a4", "quantize_weight_int4",
    "svdquant_decompose", "unpack_int4", "w4a4_int_ops", "act_quant_bytes", "svdq_pair_forward",
    "svdq_concat_forward",
]
