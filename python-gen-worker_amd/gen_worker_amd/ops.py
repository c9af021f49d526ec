"""``torch.library`` operators of the int4-g64 SVDQuant / W8A8 path.

The reference registers its fused lane as ``cozy_gen_worker::*`` custom ops
(``src/gen_worker/models/svdq_fused.py:17-19``, ``:293-389``) and its native
probe as ``cozy_kernels::probe_add_one`` (``csrc/cozy_kernels/ops.cpp:29-36``).
The same names and schemas are registered here, backed by the HIP kernels of
``libgen_worker_amd.so``, with int4 group-64 semantics in place of nvfp4:

* ``svdq_quant(x2, smooth, s2, blocked) -> (q, s)``: q uint8 [M, K/2],
  s fp16 [M, K/64]. int4 scales are flat; ``blocked=True`` (the nvfp4 cuBLAS
  tile swizzle) is refused.
* ``svdq_gemm_w4a4_lora(qa, sa, wq_kn, ws, s2, second, lora_act, up, bias)``:
  ``wq_kn`` is the reference's K-major packed weight [K/2, N].
* ``svdq_epilogue_lora(y0, la, up, s2, second, bias)``.

Additions (no reference counterpart; the fused forms the reference keeps as
separate steps):

* ``svdq_prep_proj_down(proj_down) -> proj_down_op``: proj_down [K, rank] in
  the operand order kernel 1 reads ([ceil(K/256)*256, rank], done once).
* ``svdq_quant_lora(x2, smooth, s2, proj_down_op) -> (q, s, la)``: kernel 1
  with ``la = x2 @ proj_down`` fused.
* ``svdq_quant_fp6(x2, smooth, s2, proj_down_op) -> (q6, la)``: the same
  codes and scales as fp6 operand records [K/128, M, 104] (e3m2 codes + fp16
  group scales, the fp6 GEMM's operand format; ``la`` empty when
  ``proj_down_op`` is None).
* ``svdq_pack_weight_fp6(weight, wscales)``, ``svdq_w4a4_linear_fp6(qa6,
  weight_fp6, s2, second, la, up, bias, out_dtype, gelu)``,
  ``svdq_group_psums_fp6(qa6, weight_fp6)``: the fp6 GEMM lane.
* ``svdq_w4a4_linear_fp6_next(...)`` and ``svdq_quant_fp6_accum(...)``: the
  next layer's activation quantization fused into the GEMM epilogue (fp6
  records + fp32 la accumulated), for fc1 -> GELU -> fc2 and for a layer
  whose input concatenates two producers.
* ``svdq_w4a4_linear(qa, sa, weight, wscales, s2, second, la, up, bias,
  out_dtype, gelu)``: kernel 2 on the resident ``weight`` [N, K/2] layout.
* ``svdq_group_psums(qa, qw)``: exact int32 per-group partial sums (debug).
* ``w8a8_quant(x2) -> (q, sa)`` and ``w8a8_scaled_mm(qa, weight, sa,
  weight_scale, bias, out_dtype)``: the int8 lane.

Every op runs on the current HIP stream and allocates its outputs with
``torch.empty`` on the input's device, as the reference launchers do
(``models/svdq_fused.py:260-266``). Inputs must be contiguous CUDA tensors;
CPU tensors are refused (there is no CPU implementation).
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _native as nat

GROUP = 64
FP6_STAGE = 128   # K elements per fp6 operand record


class SvdqOpError(ValueError):
    """Typed contract violation at the op boundary (never a silent fallback)."""


def _check_cuda(name: str, **tensors: Optional[Tensor]) -> None:
    for k, t in tensors.items():
        if t is None:
            continue
        if not t.is_cuda:
            raise SvdqOpError(f"{name}: {k} is on {t.device}; the int4/int8 path runs on the GPU only")
        if not t.is_contiguous():
            raise SvdqOpError(f"{name}: {k} must be contiguous")


def _check_dtype(name: str, t: Optional[Tensor], *dtypes: torch.dtype, what: str) -> None:
    if t is not None and t.dtype not in dtypes:
        raise SvdqOpError(f"{name}: {what} has dtype {t.dtype}, expected one of {dtypes}")


def _scalar_f32(name: str, s2: Optional[Tensor]) -> Optional[Tensor]:
    if s2 is None:
        return None
    if s2.numel() != 1:
        raise SvdqOpError(f"{name}: s2 must hold one value, got {s2.numel()}")
    if s2.dtype != torch.float32:
        s2 = s2.float()
    return s2.reshape(()).contiguous()


def _dt_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return nat.DT_BF16
    if dtype == torch.float16:
        return nat.DT_F16
    if dtype == torch.float32:
        return nat.DT_F32
    raise SvdqOpError(f"unsupported dtype {dtype}")


# ---------------------------------------------------------------------------
# kernel 1
# ---------------------------------------------------------------------------

def _quant_impl(x2: Tensor, smooth: Optional[Tensor], s2: Optional[Tensor], proj_down_op: Optional[Tensor],
                fmt: int = 0) -> tuple[Tensor, Tensor, Optional[Tensor]]:
    name = "svdq_quant"
    if x2.dim() != 2:
        raise SvdqOpError(f"{name}: x2 must be 2-D, got {tuple(x2.shape)}")
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_dtype(name, smooth, torch.bfloat16, what="smooth")
    _check_dtype(name, proj_down_op, torch.bfloat16, what="proj_down_op")
    s2 = _scalar_f32(name, s2)
    _check_cuda(name, x2=x2, smooth=smooth, s2=s2, proj_down_op=proj_down_op)
    m, k = int(x2.shape[0]), int(x2.shape[1])
    if k % GROUP:
        raise SvdqOpError(f"{name}: K={k} is not a multiple of {GROUP}")
    if smooth is not None and smooth.numel() != k:
        raise SvdqOpError(f"{name}: smooth has {smooth.numel()} values for K={k}")
    rank = 0
    if proj_down_op is not None:
        kp = (k + 255) // 256 * 256
        if proj_down_op.dim() != 2 or int(proj_down_op.shape[0]) != kp:
            raise SvdqOpError(f"{name}: proj_down_op must be [{kp}, rank] (svdq_prep_proj_down of a [K={k}, rank] "
                              f"proj_down), got {tuple(proj_down_op.shape)}")
        rank = int(proj_down_op.shape[1])
    x2 = x2 if x2.stride(1) == 1 else x2.contiguous()
    if fmt == nat.QFMT_FP6:
        if k % FP6_STAGE:
            raise SvdqOpError(f"{name}: the fp6 records need K % {FP6_STAGE} == 0, got K={k}")
        q = torch.empty(k // FP6_STAGE, m, nat.FP6_REC, dtype=torch.uint8, device=x2.device)
        s = None   # the records carry the scales
    else:
        q = torch.empty(m, k // 2, dtype=torch.uint8, device=x2.device)
        s = torch.empty(m, k // GROUP, dtype=torch.float16, device=x2.device)
    la = torch.empty(m, rank, dtype=torch.bfloat16, device=x2.device) if proj_down_op is not None else None
    nat.call("gwa_svdq_quant_int4", nat.ptr(x2), int(x2.stride(0)), nat.ptr(smooth), nat.ptr(s2),
             nat.ptr(proj_down_op), rank, fmt, nat.ptr(q), nat.ptr(s), nat.ptr(la), m, k, nat.stream_of(x2))
    return q, s, la


@torch.library.custom_op("cozy_gen_worker::svdq_quant", mutates_args=())
def svdq_quant(x2: Tensor, smooth: Optional[Tensor], s2: Tensor, blocked: bool) -> tuple[Tensor, Tensor]:
    """int4 group-64 activation quant: (packed codes uint8 [M, K/2], fp16 scales [M, K/64])."""
    if blocked:
        raise SvdqOpError("svdq_quant: int4 group scales are flat [M, K/64]; the blocked (cuBLAS 128x4 "
                          "tile) layout is an nvfp4 format and is not produced")
    q, s, _ = _quant_impl(x2, smooth, s2, None)
    return q, s


@svdq_quant.register_fake
def _(x2: Tensor, smooth: Optional[Tensor], s2: Tensor, blocked: bool) -> tuple[Tensor, Tensor]:
    m, k = int(x2.shape[0]), int(x2.shape[1])
    return (x2.new_empty(m, k // 2, dtype=torch.uint8), x2.new_empty(m, k // GROUP, dtype=torch.float16))


@torch.library.custom_op("cozy_gen_worker::svdq_prep_proj_down", mutates_args=())
def svdq_prep_proj_down(proj_down: Tensor) -> Tensor:
    """proj_down bf16 [K, rank] -> the operand order kernel 1 reads, [ceil(K/256)*256, rank] (zero padded)."""
    name = "svdq_prep_proj_down"
    _check_dtype(name, proj_down, torch.bfloat16, what="proj_down")
    _check_cuda(name, proj_down=proj_down)
    if proj_down.dim() != 2:
        raise SvdqOpError(f"{name}: proj_down must be [K, rank], got {tuple(proj_down.shape)}")
    k, r = int(proj_down.shape[0]), int(proj_down.shape[1])
    if k % GROUP or r not in (16, 32, 64, 128):
        raise SvdqOpError(f"{name}: K={k} must be a multiple of {GROUP} and rank={r} in (16, 32, 64, 128)")
    out = torch.empty((k + 255) // 256 * 256, r, dtype=torch.bfloat16, device=proj_down.device)
    nat.call("gwa_svdq_prep_proj_down", nat.ptr(proj_down.contiguous()), nat.ptr(out), k, r,
             nat.stream_of(proj_down))
    return out


@svdq_prep_proj_down.register_fake
def _(proj_down):
    k, r = int(proj_down.shape[0]), int(proj_down.shape[1])
    return proj_down.new_empty((k + 255) // 256 * 256, r)


@torch.library.custom_op("cozy_gen_worker::svdq_quant_lora", mutates_args=())
def svdq_quant_lora(x2: Tensor, smooth: Optional[Tensor], s2: Optional[Tensor],
                    proj_down_op: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Kernel 1 with the low-rank down-projection fused: (q, s, la = x2 @ proj_down)."""
    q, s, la = _quant_impl(x2, smooth, s2, proj_down_op)
    assert la is not None
    return q, s, la


@svdq_quant_lora.register_fake
def _(x2, smooth, s2, proj_down_op):
    m, k = int(x2.shape[0]), int(x2.shape[1])
    r = int(proj_down_op.shape[1])
    return (x2.new_empty(m, k // 2, dtype=torch.uint8), x2.new_empty(m, k // GROUP, dtype=torch.float16),
            x2.new_empty(m, r, dtype=torch.bfloat16))


@torch.library.custom_op("cozy_gen_worker::svdq_quant_fp6", mutates_args=())
def svdq_quant_fp6(x2: Tensor, smooth: Optional[Tensor], s2: Optional[Tensor],
                   proj_down_op: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """Kernel 1 writing fp6 operand records [K/128, M, 104] (e3m2 codes + the fp16 group scales: the fp6
    GEMM's operand format); returns ``(records, la)``, la [M, 0] when ``proj_down_op`` is None."""
    q, _, la = _quant_impl(x2, smooth, s2, proj_down_op, nat.QFMT_FP6)
    if la is None:
        la = x2.new_empty(int(x2.shape[0]), 0)
    return q, la


@svdq_quant_fp6.register_fake
def _(x2, smooth, s2, proj_down_op):
    m, k = int(x2.shape[0]), int(x2.shape[1])
    r = int(proj_down_op.shape[1]) if proj_down_op is not None else 0
    return (x2.new_empty(k // FP6_STAGE, m, nat.FP6_REC, dtype=torch.uint8), x2.new_empty(m, r, dtype=torch.bfloat16))


# ---------------------------------------------------------------------------
# kernel 2
# ---------------------------------------------------------------------------

def _gemm_impl(qa: Tensor, sa: Tensor, weight: Tensor, wscales: Tensor, s2: Optional[Tensor],
               second: Optional[Tensor], la: Optional[Tensor], up: Optional[Tensor], bias: Optional[Tensor],
               out_dtype: torch.dtype, gelu: bool) -> Tensor:
    name = "svdq_w4a4_linear"
    s2 = _scalar_f32(name, s2)
    if second is not None and second.dtype != torch.float32:
        second = second.float().contiguous()
    _check_dtype(name, qa, torch.uint8, what="qa")
    _check_dtype(name, weight, torch.uint8, what="weight")
    _check_dtype(name, sa, torch.float16, what="sa")
    _check_dtype(name, wscales, torch.float16, what="weight scales")
    _check_dtype(name, la, torch.bfloat16, what="la")
    _check_dtype(name, up, torch.bfloat16, what="up")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    _check_cuda(name, qa=qa, sa=sa, weight=weight, wscales=wscales, s2=s2, second=second, la=la, up=up, bias=bias)
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise SvdqOpError(f"{name}: out_dtype {out_dtype} not bf16/fp16")
    m, kh = int(qa.shape[0]), int(qa.shape[1])
    k = 2 * kh
    n = int(weight.shape[0])
    if tuple(weight.shape) != (n, kh):
        raise SvdqOpError(f"{name}: weight {tuple(weight.shape)} != [N, K/2={kh}]")
    if tuple(sa.shape) != (m, k // GROUP) or tuple(wscales.shape) != (n, k // GROUP):
        raise SvdqOpError(f"{name}: scales {tuple(sa.shape)} / {tuple(wscales.shape)} do not match "
                          f"[M, K/64] / [N, K/64] for M={m} N={n} K={k}")
    if (la is None) != (up is None):
        raise SvdqOpError(f"{name}: la and up must both be given or both be None")
    rank = 0
    if la is not None:
        rank = int(up.shape[1])
        if tuple(la.shape) != (m, rank) or tuple(up.shape) != (n, rank):
            raise SvdqOpError(f"{name}: la {tuple(la.shape)} / up {tuple(up.shape)} do not match rank {rank}")
    if bias is not None and bias.numel() != n:
        raise SvdqOpError(f"{name}: bias has {bias.numel()} values for N={n}")
    sec_n = 0 if second is None else int(second.numel())
    out = torch.empty(m, n, dtype=out_dtype, device=qa.device)
    nat.call("gwa_svdq_gemm_w4a4", nat.ptr(qa), nat.ptr(sa), nat.ptr(weight), nat.ptr(wscales), nat.ptr(s2),
             nat.ptr(second), sec_n, nat.ptr(la), nat.ptr(up), rank, nat.ptr(bias), nat.ptr(out),
             _dt_code(out_dtype), nat.EPI_GELU_TANH if gelu else 0, m, n, k, nat.stream_of(qa))
    return out


@torch.library.custom_op("cozy_gen_worker::svdq_w4a4_linear", mutates_args=())
def svdq_w4a4_linear(qa: Tensor, sa: Tensor, weight: Tensor, wscales: Tensor, s2: Optional[Tensor],
                     second: Optional[Tensor], la: Optional[Tensor], up: Optional[Tensor],
                     bias: Optional[Tensor], out_dtype: torch.dtype, gelu: bool) -> Tensor:
    """W4A4 GEMM + fused epilogue on the resident [N, K/2] weight layout."""
    return _gemm_impl(qa, sa, weight, wscales, s2, second, la, up, bias, out_dtype, gelu)


@svdq_w4a4_linear.register_fake
def _(qa, sa, weight, wscales, s2, second, la, up, bias, out_dtype, gelu):
    return qa.new_empty(int(qa.shape[0]), int(weight.shape[0]), dtype=out_dtype)


def _epilogue_operands(name: str, m: int, n: int, la: Optional[Tensor], up: Optional[Tensor],
                       bias: Optional[Tensor], second: Optional[Tensor]) -> tuple[int, int]:
    """Shape checks of the fused epilogue's operands; returns (rank, second_numel)."""
    if (la is None) != (up is None):
        raise SvdqOpError(f"{name}: la and up must both be given or both be None")
    rank = 0
    if la is not None:
        rank = int(up.shape[1])
        if tuple(la.shape) != (m, rank) or tuple(up.shape) != (n, rank):
            raise SvdqOpError(f"{name}: la {tuple(la.shape)} / up {tuple(up.shape)} do not match rank {rank}")
    if bias is not None and bias.numel() != n:
        raise SvdqOpError(f"{name}: bias has {bias.numel()} values for N={n}")
    return rank, (0 if second is None else int(second.numel()))


def _fp6_records_k(name: str, rec: Tensor, what: str) -> tuple[int, int]:
    """(rows, K) of an fp6 operand record tensor [K/128, rows, 104]."""
    if rec.dim() != 3 or int(rec.shape[2]) != nat.FP6_REC:
        raise SvdqOpError(f"{name}: {what} must be fp6 records [K/{FP6_STAGE}, rows, {nat.FP6_REC}], "
                          f"got {tuple(rec.shape)}")
    return int(rec.shape[1]), int(rec.shape[0]) * FP6_STAGE


def _fp6_impl(qa6: Tensor, weight_fp6: Tensor, s2: Optional[Tensor], second: Optional[Tensor],
              la: Optional[Tensor], up: Optional[Tensor], bias: Optional[Tensor], out_dtype: torch.dtype,
              gelu: bool) -> Tensor:
    name = "svdq_w4a4_linear_fp6"
    s2 = _scalar_f32(name, s2)
    if second is not None and second.dtype != torch.float32:
        second = second.float().contiguous()
    _check_dtype(name, qa6, torch.uint8, what="qa6")
    _check_dtype(name, weight_fp6, torch.uint8, what="weight_fp6")
    _check_dtype(name, la, torch.bfloat16, what="la")
    _check_dtype(name, up, torch.bfloat16, what="up")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    _check_cuda(name, qa6=qa6, weight_fp6=weight_fp6, s2=s2, second=second, la=la, up=up, bias=bias)
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise SvdqOpError(f"{name}: out_dtype {out_dtype} not bf16/fp16")
    m, k = _fp6_records_k(name, qa6, "qa6")
    n, kw = _fp6_records_k(name, weight_fp6, "weight_fp6")
    if kw != k:
        raise SvdqOpError(f"{name}: activation K={k} and weight K={kw} differ")
    rank, sec_n = _epilogue_operands(name, m, n, la, up, bias, second)
    out = torch.empty(m, n, dtype=out_dtype, device=qa6.device)
    nat.call("gwa_svdq_gemm_w4a4_fp6", nat.ptr(qa6), nat.ptr(weight_fp6.contiguous()), nat.ptr(s2), nat.ptr(second),
             sec_n, nat.ptr(la), nat.ptr(up), rank, nat.ptr(bias), nat.ptr(out), _dt_code(out_dtype),
             nat.EPI_GELU_TANH if gelu else 0, m, n, k, nat.stream_of(qa6))
    return out


@torch.library.custom_op("cozy_gen_worker::svdq_w4a4_linear_fp6", mutates_args=())
def svdq_w4a4_linear_fp6(qa6: Tensor, weight_fp6: Tensor, s2: Optional[Tensor], second: Optional[Tensor],
                         la: Optional[Tensor], up: Optional[Tensor], bias: Optional[Tensor], out_dtype: torch.dtype,
                         gelu: bool) -> Tensor:
    """W4A4 GEMM + fused epilogue on fp6 operand records (``svdq_quant_fp6`` activations,
    ``svdq_pack_weight_fp6`` weights)."""
    return _fp6_impl(qa6, weight_fp6, s2, second, la, up, bias, out_dtype, gelu)


@svdq_w4a4_linear_fp6.register_fake
def _(qa6, weight_fp6, s2, second, la, up, bias, out_dtype, gelu):
    return qa6.new_empty(int(qa6.shape[1]), int(weight_fp6.shape[1]), dtype=out_dtype)


def _next_records(name: str, q6: Tensor, m: int, k: int, stage_offset: int) -> int:
    """Checks a record buffer [S, m, 104] that receives stages [stage_offset, stage_offset + k/128); returns the
    byte address of the first of them."""
    _check_dtype(name, q6, torch.uint8, what="records")
    rows, ktot = _fp6_records_k(name, q6, "records")
    if rows != m:
        raise SvdqOpError(f"{name}: records hold {rows} rows, the activations {m}")
    if stage_offset < 0 or stage_offset * FP6_STAGE + k > ktot:
        raise SvdqOpError(f"{name}: stages [{stage_offset}, {stage_offset + k // FP6_STAGE}) do not fit records "
                          f"of {ktot // FP6_STAGE} stages")
    return q6.data_ptr() + stage_offset * m * nat.FP6_REC


def _next_lowrank(name: str, proj_down_op: Optional[Tensor], la32: Optional[Tensor], m: int, k: int) -> int:
    """Checks the next layer's (proj_down_op rows for these k columns, fp32 la accumulator); returns the rank."""
    if (proj_down_op is None) != (la32 is None):
        raise SvdqOpError(f"{name}: proj_down_op and la32 must both be given or both be None")
    if proj_down_op is None:
        return 0
    _check_dtype(name, proj_down_op, torch.bfloat16, what="proj_down_op")
    _check_dtype(name, la32, torch.float32, what="la32")
    r = int(la32.shape[1]) if la32.dim() == 2 else -1
    if la32.dim() != 2 or int(la32.shape[0]) != m:
        raise SvdqOpError(f"{name}: la32 must be [{m}, rank], got {tuple(la32.shape)}")
    if proj_down_op.dim() != 2 or int(proj_down_op.shape[1]) != r or int(proj_down_op.shape[0]) < k:
        raise SvdqOpError(f"{name}: proj_down_op must be [>= {k}, {r}] rows in operand order, got "
                          f"{tuple(proj_down_op.shape)}")
    return r


@torch.library.custom_op("cozy_gen_worker::svdq_w4a4_linear_fp6_next", mutates_args=("next_q6", "next_la32"))
def svdq_w4a4_linear_fp6_next(qa6: Tensor, weight_fp6: Tensor, s2: Optional[Tensor], second: Optional[Tensor],
                              la: Optional[Tensor], up: Optional[Tensor], bias: Optional[Tensor], gelu: bool,
                              next_smooth: Optional[Tensor], next_proj_down_op: Optional[Tensor], next_q6: Tensor,
                              next_la32: Optional[Tensor], stage_offset: int, write_out: bool) -> Tensor:
    """W4A4 GEMM whose epilogue also quantizes its bf16 output as the NEXT layer's input: writes that layer's
    fp6 records into stages ``stage_offset ..`` of ``next_q6`` [S, M, 104] (bit-identical to ``svdq_quant_fp6``
    on the output with ``next_smooth``) and adds ``output @ proj_down_next`` into ``next_la32`` fp32 [M, r]
    (atomic adds over column tiles). ``next_proj_down_op`` holds the next layer's proj_down rows for these N
    columns in operand order (a prefix-aligned slice of its ``proj_down_op``). Returns the bf16 output
    [M, N] when ``write_out``, else an empty [M, 0]."""
    name = "svdq_w4a4_linear_fp6_next"
    s2 = _scalar_f32(name, s2)
    if second is not None and second.dtype != torch.float32:
        second = second.float().contiguous()
    _check_dtype(name, qa6, torch.uint8, what="qa6")
    _check_dtype(name, weight_fp6, torch.uint8, what="weight_fp6")
    _check_dtype(name, la, torch.bfloat16, what="la")
    _check_dtype(name, up, torch.bfloat16, what="up")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    _check_dtype(name, next_smooth, torch.bfloat16, what="next_smooth")
    _check_cuda(name, qa6=qa6, weight_fp6=weight_fp6, s2=s2, second=second, la=la, up=up, bias=bias,
                next_smooth=next_smooth, next_proj_down_op=next_proj_down_op, next_q6=next_q6, next_la32=next_la32)
    m, k = _fp6_records_k(name, qa6, "qa6")
    n, kw = _fp6_records_k(name, weight_fp6, "weight_fp6")
    if kw != k:
        raise SvdqOpError(f"{name}: activation K={k} and weight K={kw} differ")
    if n % FP6_STAGE:
        raise SvdqOpError(f"{name}: N={n} is not a multiple of {FP6_STAGE} (whole stages of the next layer)")
    if next_smooth is not None and next_smooth.numel() != n:
        raise SvdqOpError(f"{name}: next_smooth has {next_smooth.numel()} values for N={n}")
    rank, sec_n = _epilogue_operands(name, m, n, la, up, bias, second)
    q6_addr = _next_records(name, next_q6, m, n, stage_offset)
    nrank = _next_lowrank(name, next_proj_down_op, next_la32, m, n)
    out = torch.empty(m, n if write_out else 0, dtype=torch.bfloat16, device=qa6.device)
    nat.call("gwa_svdq_gemm_w4a4_fp6_next", nat.ptr(qa6), nat.ptr(weight_fp6), nat.ptr(s2), nat.ptr(second),
             sec_n, nat.ptr(la), nat.ptr(up), rank, nat.ptr(bias), nat.ptr(out) if write_out else None,
             nat.EPI_GELU_TANH if gelu else 0, nat.ptr(next_smooth), nat.ptr(next_proj_down_op), nrank, q6_addr,
             nat.ptr(next_la32), m, n, k, nat.stream_of(qa6))
    return out


@svdq_w4a4_linear_fp6_next.register_fake
def _(qa6, weight_fp6, s2, second, la, up, bias, gelu, next_smooth, next_proj_down_op, next_q6, next_la32,
      stage_offset, write_out):
    return qa6.new_empty(int(qa6.shape[1]), int(weight_fp6.shape[1]) if write_out else 0, dtype=torch.bfloat16)


@torch.library.custom_op("cozy_gen_worker::svdq_quant_fp6_accum", mutates_args=("q6", "la32"))
def svdq_quant_fp6_accum(x2: Tensor, smooth: Optional[Tensor], proj_down_op: Optional[Tensor], q6: Tensor,
                         la32: Optional[Tensor]) -> None:
    """Kernel 1 into stages [0, K/128) of the record buffer ``q6`` [S, M, 104] with ``la32`` fp32 [M, r]
    += x2 @ proj_down (``proj_down_op``: the consumer's operand-order proj_down rows for these K columns).
    With ``svdq_w4a4_linear_fp6_next`` writing the later stages it builds the input of a layer that takes
    a concatenation [x2, producer output]."""
    name = "svdq_quant_fp6_accum"
    if x2.dim() != 2:
        raise SvdqOpError(f"{name}: x2 must be 2-D, got {tuple(x2.shape)}")
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_dtype(name, smooth, torch.bfloat16, what="smooth")
    _check_cuda(name, x2=x2, smooth=smooth, proj_down_op=proj_down_op, q6=q6, la32=la32)
    m, k = int(x2.shape[0]), int(x2.shape[1])
    if k % FP6_STAGE:
        raise SvdqOpError(f"{name}: the fp6 records need K % {FP6_STAGE} == 0, got K={k}")
    if smooth is not None and smooth.numel() != k:
        raise SvdqOpError(f"{name}: smooth has {smooth.numel()} values for K={k}")
    q6_addr = _next_records(name, q6, m, k, 0)
    rank = _next_lowrank(name, proj_down_op, la32, m, k)
    if proj_down_op is not None and int(proj_down_op.shape[0]) < (k + 255) // 256 * 256:
        raise SvdqOpError(f"{name}: proj_down_op needs {(k + 255) // 256 * 256} rows for K={k}")
    nat.call("gwa_svdq_quant_fp6_la_f32", nat.ptr(x2), int(x2.stride(0)), nat.ptr(smooth), nat.ptr(proj_down_op),
             rank, q6_addr, nat.ptr(la32), m, k, nat.stream_of(x2))


@svdq_quant_fp6_accum.register_fake
def _(x2, smooth, proj_down_op, q6, la32):
    return None


@torch.library.custom_op("cozy_gen_worker::svdq_pack_weight_fp6", mutates_args=())
def svdq_pack_weight_fp6(weight: Tensor, wscales: Tensor) -> Tensor:
    """Logical int4 weights [N, K/2] + fp16 group scales [N, K/64] -> fp6 operand records
    [K/128, N, 104] (any code in [-8, 7])."""
    name = "svdq_pack_weight_fp6"
    _check_dtype(name, weight, torch.uint8, what="weight")
    _check_dtype(name, wscales, torch.float16, what="wscales")
    _check_cuda(name, weight=weight, wscales=wscales)
    n, kh = int(weight.shape[0]), int(weight.shape[1])
    k = 2 * kh
    if k % FP6_STAGE:
        raise SvdqOpError(f"{name}: K={k} is not a multiple of {FP6_STAGE}")
    if tuple(wscales.shape) != (n, k // GROUP):
        raise SvdqOpError(f"{name}: wscales {tuple(wscales.shape)} do not match [N={n}, K/64={k // GROUP}]")
    out = torch.empty(k // FP6_STAGE, n, nat.FP6_REC, dtype=torch.uint8, device=weight.device)
    nat.call("gwa_svdq_pack_weight_fp6", nat.ptr(weight.contiguous()), nat.ptr(wscales.contiguous()), nat.ptr(out),
             n, k, nat.stream_of(weight))
    return out


@svdq_pack_weight_fp6.register_fake
def _(weight, wscales):
    return weight.new_empty(int(weight.shape[1]) * 2 // FP6_STAGE, int(weight.shape[0]), nat.FP6_REC)


@torch.library.custom_op("cozy_gen_worker::svdq_group_psums_fp6", mutates_args=())
def svdq_group_psums_fp6(qa6: Tensor, weight_fp6: Tensor) -> Tensor:
    """Exact int32 [M, N, K/64] per-group partial sums through the fp6 GEMM's MFMA (debug)."""
    name = "svdq_group_psums_fp6"
    _check_dtype(name, qa6, torch.uint8, what="qa6")
    _check_dtype(name, weight_fp6, torch.uint8, what="weight_fp6")
    _check_cuda(name, qa6=qa6, weight_fp6=weight_fp6)
    m, k = _fp6_records_k(name, qa6, "qa6")
    n, kw = _fp6_records_k(name, weight_fp6, "weight_fp6")
    if kw != k:
        raise SvdqOpError(f"{name}: activation K={k} and weight K={kw} differ")
    out = torch.empty(m, n, k // GROUP, dtype=torch.int32, device=qa6.device)
    nat.call("gwa_svdq_group_psums_fp6", nat.ptr(qa6.contiguous()), nat.ptr(weight_fp6.contiguous()), nat.ptr(out),
             m, n, k, nat.stream_of(qa6))
    return out


@svdq_group_psums_fp6.register_fake
def _(qa6, weight_fp6):
    return qa6.new_empty(int(qa6.shape[1]), int(weight_fp6.shape[1]), int(qa6.shape[0]) * FP6_STAGE // GROUP,
                         dtype=torch.int32)


@torch.library.custom_op("cozy_gen_worker::svdq_gemm_w4a4_lora", mutates_args=())
def svdq_gemm_w4a4_lora(qa: Tensor, sa: Tensor, wq_kn: Tensor, ws: Tensor, s2: Tensor, second: Tensor,
                        lora_act: Tensor, up: Tensor, bias: Optional[Tensor]) -> Tensor:
    """The reference schema (``models/svdq_fused.py:379-389``): K-major weight ``wq_kn`` [K/2, N], bf16 out."""
    _check_cuda("svdq_gemm_w4a4_lora", wq_kn=wq_kn)
    _check_dtype("svdq_gemm_w4a4_lora", wq_kn, torch.uint8, what="wq_kn")
    kh, n = int(wq_kn.shape[0]), int(wq_kn.shape[1])
    w_nk = torch.empty(n, kh, dtype=torch.uint8, device=wq_kn.device)
    nat.call("gwa_transpose_2d", nat.ptr(wq_kn), nat.ptr(w_nk), kh, n, 1, nat.stream_of(wq_kn))
    return _gemm_impl(qa, sa, w_nk, ws, s2, second, lora_act, up, bias, torch.bfloat16, False)


@svdq_gemm_w4a4_lora.register_fake
def _(qa, sa, wq_kn, ws, s2, second, lora_act, up, bias):
    return qa.new_empty(int(qa.shape[0]), int(wq_kn.shape[1]), dtype=torch.bfloat16)


@torch.library.custom_op("cozy_gen_worker::svdq_epilogue_lora", mutates_args=())
def svdq_epilogue_lora(y0: Tensor, la: Tensor, up: Tensor, s2: Tensor, second: Tensor,
                       bias: Optional[Tensor]) -> Tensor:
    """``y0 * (s2 * second) + la @ up^T + bias`` -> bf16 (``models/svdq_fused.py:315-377``)."""
    name = "svdq_epilogue_lora"
    s2 = _scalar_f32(name, s2)
    if second.dtype != torch.float32:
        second = second.float().contiguous()
    _check_dtype(name, y0, torch.bfloat16, what="y0")
    _check_dtype(name, la, torch.bfloat16, what="la")
    _check_dtype(name, up, torch.bfloat16, what="up")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    _check_cuda(name, y0=y0, la=la, up=up, s2=s2, second=second, bias=bias)
    m, n = int(y0.shape[0]), int(y0.shape[1])
    r = int(up.shape[1])
    if tuple(la.shape) != (m, r) or int(up.shape[0]) != n:
        raise SvdqOpError(f"{name}: la {tuple(la.shape)} / up {tuple(up.shape)} do not match y0 {tuple(y0.shape)}")
    out = torch.empty(m, n, dtype=torch.bfloat16, device=y0.device)
    nat.call("gwa_svdq_epilogue_lora", nat.ptr(y0), nat.ptr(la), nat.ptr(up), r, nat.ptr(s2), nat.ptr(second),
             int(second.numel()), nat.ptr(bias), nat.ptr(out), m, n, nat.stream_of(y0))
    return out


@svdq_epilogue_lora.register_fake
def _(y0, la, up, s2, second, bias):
    return y0.new_empty(int(y0.shape[0]), int(y0.shape[1]), dtype=torch.bfloat16)


@torch.library.custom_op("cozy_gen_worker::svdq_group_psums", mutates_args=())
def svdq_group_psums(qa: Tensor, qw: Tensor) -> Tensor:
    """Exact int32 [M, N, K/64] per-group partial sums (debug/parity entry)."""
    name = "svdq_group_psums"
    _check_dtype(name, qa, torch.uint8, what="qa")
    _check_dtype(name, qw, torch.uint8, what="qw")
    _check_cuda(name, qa=qa, qw=qw)
    m, kh = int(qa.shape[0]), int(qa.shape[1])
    n = int(qw.shape[0])
    if int(qw.shape[1]) != kh:
        raise SvdqOpError(f"{name}: qa {tuple(qa.shape)} and qw {tuple(qw.shape)} disagree on K/2")
    out = torch.empty(m, n, (2 * kh) // GROUP, dtype=torch.int32, device=qa.device)
    nat.call("gwa_svdq_group_psums", nat.ptr(qa), nat.ptr(qw), nat.ptr(out), m, n, 2 * kh, nat.stream_of(qa))
    return out


@svdq_group_psums.register_fake
def _(qa, qw):
    return qa.new_empty(int(qa.shape[0]), int(qw.shape[0]), (2 * int(qa.shape[1])) // GROUP, dtype=torch.int32)


# ---------------------------------------------------------------------------
# W8A8
# ---------------------------------------------------------------------------

@torch.library.custom_op("cozy_gen_worker::w8a8_quant", mutates_args=())
def w8a8_quant(x2: Tensor) -> tuple[Tensor, Tensor]:
    """Per-token int8: (q int8 [M, K], sa fp32 [M, 1])."""
    name = "w8a8_quant"
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_cuda(name, x2=x2)
    m, k = int(x2.shape[0]), int(x2.shape[1])
    q = torch.empty(m, k, dtype=torch.int8, device=x2.device)
    sa = torch.empty(m, 1, dtype=torch.float32, device=x2.device)
    nat.call("gwa_w8a8_quant_int8", nat.ptr(x2), k, nat.ptr(q), nat.ptr(sa), m, k, nat.stream_of(x2))
    return q, sa


@w8a8_quant.register_fake
def _(x2):
    m, k = int(x2.shape[0]), int(x2.shape[1])
    return x2.new_empty(m, k, dtype=torch.int8), x2.new_empty(m, 1, dtype=torch.float32)


@torch.library.custom_op("cozy_gen_worker::w8a8_scaled_mm", mutates_args=())
def w8a8_scaled_mm(qa: Tensor, weight: Tensor, sa: Tensor, weight_scale: Tensor, bias: Optional[Tensor],
                   out_dtype: torch.dtype) -> Tensor:
    """``_scaled_mm(qa, weight.t(), scale_a=sa, scale_b=weight_scale.t(), bias, out_dtype)`` on int8 codes."""
    name = "w8a8_scaled_mm"
    _check_dtype(name, qa, torch.int8, what="qa")
    _check_dtype(name, weight, torch.int8, what="weight")
    _check_dtype(name, sa, torch.float32, what="sa")
    _check_dtype(name, weight_scale, torch.float32, what="weight_scale")
    _check_dtype(name, bias, torch.float32, torch.bfloat16, torch.float16, what="bias")
    _check_cuda(name, qa=qa, weight=weight, sa=sa, weight_scale=weight_scale, bias=bias)
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise SvdqOpError(f"{name}: out_dtype {out_dtype} not bf16/fp16")
    m, k = int(qa.shape[0]), int(qa.shape[1])
    n = int(weight.shape[0])
    if int(weight.shape[1]) != k or sa.numel() != m or weight_scale.numel() != n:
        raise SvdqOpError(f"{name}: shapes qa {tuple(qa.shape)} weight {tuple(weight.shape)} sa {tuple(sa.shape)} "
                          f"weight_scale {tuple(weight_scale.shape)} disagree")
    if bias is not None and bias.numel() != n:
        raise SvdqOpError(f"{name}: bias has {bias.numel()} values for N={n}")
    out = torch.empty(m, n, dtype=out_dtype, device=qa.device)
    nat.call("gwa_w8a8_gemm", nat.ptr(qa), nat.ptr(weight), nat.ptr(sa), nat.ptr(weight_scale), nat.ptr(bias),
             _dt_code(bias.dtype) if bias is not None else 0, nat.ptr(out), _dt_code(out_dtype), m, n, k,
             nat.stream_of(qa))
    return out


@w8a8_scaled_mm.register_fake
def _(qa, weight, sa, weight_scale, bias, out_dtype):
    return qa.new_empty(int(qa.shape[0]), int(weight.shape[0]), dtype=out_dtype)


# ---------------------------------------------------------------------------
# cozy_kernels probe (csrc/cozy_kernels/ops.cpp:29-36)
# ---------------------------------------------------------------------------

@torch.library.custom_op("cozy_kernels::probe_add_one", mutates_args=())
def probe_add_one(x: Tensor) -> Tensor:
    if not (x.is_cuda and x.dtype == torch.float32):
        raise SvdqOpError("probe_add_one expects a float32 CUDA tensor")
    xin = x.contiguous()
    out = torch.empty_like(xin)
    nat.call("gwa_probe_add_one", nat.ptr(xin), nat.ptr(out), xin.numel(), nat.stream_of(xin))
    return out


@probe_add_one.register_fake
def _(x):
    return torch.empty_like(x)


def build_info() -> str:
    """Library build description (``cozy_kernels::build_info``, ``csrc/cozy_kernels/ops.cpp:23-27``)."""
    return f"torch={torch.__version__} {nat.build_info()}"
