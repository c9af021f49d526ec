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
* ``svdq_prep_proj_down_fp6(proj_down)`` and ``svdq_quant_fp6(x2, smooth,
  s2, proj_down_op6) -> (q6, la)``: the same codes and scales as fp6
  operand records [K/128, M, 104] (e3m2 codes + fp16 group scales, the fp6
  GEMM's operand format) and the bf16 la ([M, 0] when ``proj_down_op6`` is
  None); the fp6 GEMM takes la in bf16 or fp32.
* ``svdq_pack_weight_fp6(weight, wscales)``, ``svdq_w4a4_linear_fp6(qa6,
  weight_fp6, s2, second, la, up, bias, out_dtype, gelu)``,
  ``svdq_group_psums_fp6(qa6, weight_fp6)``: the fp6 GEMM lane.
* ``svdq_w4a4_linear_fp6_next(...)``, ``svdq_quant_fp6_into(...)`` and
  ``svdq_la_reduce(la_part)``: the next layer's activation quantization
  fused into the GEMM epilogue (fp6 records + fp32 la partial slots, summed
  in a fixed order), for fc1 -> GELU -> fc2 and for a layer whose input
  concatenates two producers.
* ``svdq_w4a4_linear(qa, sa, weight, wscales, s2, second, la, up, bias,
  out_dtype, gelu)``: kernel 2 on the resident ``weight`` [N, K/2] layout.
* ``svdq_group_psums(qa, qw)``: exact int32 per-group partial sums (debug).
* ``w8a8_quant(x2, pertensor=False, static=None) -> (q, sa)`` and
  ``w8a8_scaled_mm(qa, weight, sa, weight_scale, bias, out_dtype)``: the int8
  lane, in the reference's rowwise, pertensor and static-scale modes.
* ``awq_w4a16_mm(x2, weight, wscales, wzeros, bias)``: the reference's packed
  AWQ W4A16 op (``models/svdq_awq_packed.py:48-115``, same name and schema)
  for the M = 1 modulation layers, and ``awq_w4a16_dequant(weight, wscales,
  wzeros)``: its weight as bf16.

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


def fp6_stages(k: int) -> int:
    """Stages of fp6 records for K inputs (K % 64 == 0): with K % 128 == 64 the last is a half stage whose
    second group holds zero codes."""
    return (int(k) + FP6_STAGE - 1) // FP6_STAGE


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

def _quant_impl(x2: Tensor, smooth: Optional[Tensor], s2: Optional[Tensor],
                proj_down_op: Optional[Tensor]) -> tuple[Tensor, Tensor, Optional[Tensor]]:
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
    q = torch.empty(m, k // 2, dtype=torch.uint8, device=x2.device)
    s = torch.empty(m, k // GROUP, dtype=torch.float16, device=x2.device)
    la = torch.empty(m, rank, dtype=torch.bfloat16, device=x2.device) if proj_down_op is not None else None
    nat.call("gwa_svdq_quant_int4", nat.ptr(x2), int(x2.stride(0)), nat.ptr(smooth), nat.ptr(s2),
             nat.ptr(proj_down_op), rank, nat.QFMT_INT4, nat.ptr(q), nat.ptr(s), nat.ptr(la), m, k,
             nat.stream_of(x2))
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


RECORD_SLACK = 1024  # readable bytes after every fp6 record buffer the GEMM reads


def records_empty(stages: int, rows: int, device) -> Tensor:
    """An uninitialised fp6 record buffer [stages, rows, 104] whose storage runs 1 KB past its end: the fp6
    GEMM copies operand records in 1 KB runs and the run that holds a tile's last real row may reach up to
    1 KB past it, so every record buffer it reads (activations and weights) is allocated here."""
    n = stages * rows * nat.FP6_REC
    return torch.empty(n + RECORD_SLACK, dtype=torch.uint8, device=device)[:n].view(stages, rows, nat.FP6_REC)


def record_slack_bytes(rec: Tensor) -> int:
    """Readable bytes of ``rec``'s storage past its last element."""
    end = (rec.storage_offset() + rec.numel()) * rec.element_size()
    return rec.untyped_storage().nbytes() - end


def readable_bytes(t: Tensor) -> int:
    """Bytes of ``t``'s storage from its first element to the storage's end: the byte count the C-ABI's record
    entry points take beside each record pointer (they check the records plus the slack against it)."""
    return t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()


def _check_record_slack(name: str, rec: Tensor, what: str) -> None:
    """The fp6 GEMM copies operand records in 1 KB runs with unchecked scalar offsets: the run holding a tile's
    last real row may read up to RECORD_SLACK bytes past the last record, so a record tensor handed to it must own
    that much storage after its end (``records_empty`` allocates it; a ``clone()``, ``.to()`` copy or
    deserialized tensor does not)."""
    slack = record_slack_bytes(rec)
    if slack < RECORD_SLACK:
        raise SvdqOpError(f"{name}: {what} has {slack} readable bytes past its last record, the fp6 GEMM needs "
                          f"{RECORD_SLACK} (allocate record buffers with ops.records_empty)")


def la_partials_quant(m: int, k: int, rank: int) -> int:
    """la partial slots the fp6 act-quant kernel writes for [m, k] at this rank."""
    return int(nat.load().gwa_svdq_quant_fp6_partials(m, k, rank))


def la_partials_next(m: int, n: int) -> int:
    """la partial slots the next-layer GEMM epilogue writes for m rows and n outputs."""
    return int(nat.load().gwa_svdq_gemm_w4a4_fp6_next_partials(m, n))


def _la_part_check(name: str, la_part: Optional[Tensor], proj_down_op6: Optional[Tensor], m: int, k: int,
                   slots: int) -> int:
    """Checks a partial-slot buffer [>= slots, m, rank] and the operand-order proj_down rows for k inputs; returns
    the rank (0 without a low-rank branch)."""
    if (proj_down_op6 is None) != (la_part is None):
        raise SvdqOpError(f"{name}: proj_down_op6 and la_part must both be given or both be None")
    if proj_down_op6 is None:
        return 0
    _check_dtype(name, proj_down_op6, torch.bfloat16, what="proj_down_op6")
    _check_dtype(name, la_part, torch.float32, what="la_part")
    if la_part.dim() != 3 or int(la_part.shape[1]) != m or int(la_part.shape[0]) < slots:
        raise SvdqOpError(f"{name}: la_part must be [>= {slots}, {m}, rank], got {tuple(la_part.shape)}")
    r = int(la_part.shape[2])
    kp = fp6_stages(k) * FP6_STAGE
    if proj_down_op6.dim() != 2 or int(proj_down_op6.shape[1]) != r or int(proj_down_op6.shape[0]) < kp:
        raise SvdqOpError(f"{name}: proj_down_op6 must be [>= {kp}, {r}] rows in operand order, got "
                          f"{tuple(proj_down_op6.shape)}")
    return r


def _fp6_quant_into(name: str, x2: Tensor, smooth: Optional[Tensor], s2: Optional[Tensor],
                    proj_down_op6: Optional[Tensor], q6: Tensor, la_part: Optional[Tensor]) -> None:
    """Checks and the launch of the fp6-record act-quant kernel into stages [0, K/128) of ``q6`` and the first
    partial slots of ``la_part``."""
    if x2.dim() != 2:
        raise SvdqOpError(f"{name}: x2 must be 2-D, got {tuple(x2.shape)}")
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_dtype(name, smooth, torch.bfloat16, what="smooth")
    s2 = _scalar_f32(name, s2)
    _check_cuda(name, x2=x2, smooth=smooth, s2=s2, proj_down_op6=proj_down_op6, q6=q6, la_part=la_part)
    m, k = int(x2.shape[0]), int(x2.shape[1])
    if k % GROUP:
        raise SvdqOpError(f"{name}: the fp6 records need K % {GROUP} == 0, got K={k}")
    if k % FP6_STAGE and fp6_stages(k) != int(q6.shape[0]):
        raise SvdqOpError(f"{name}: K={k} ends in a half stage, which must be the records' last "
                          f"({int(q6.shape[0])} stages)")
    if smooth is not None and smooth.numel() != k:
        raise SvdqOpError(f"{name}: smooth has {smooth.numel()} values for K={k}")
    q6_addr = _next_records(name, q6, m, k, 0)
    r = int(la_part.shape[2]) if la_part is not None and la_part.dim() == 3 else 0
    rank = _la_part_check(name, la_part, proj_down_op6, m, k, la_partials_quant(m, k, r) if r else 0)
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    nat.call("gwa_svdq_quant_fp6", nat.ptr(x2), int(x2.stride(0)), nat.ptr(smooth), nat.ptr(s2),
             nat.ptr(proj_down_op6), rank, q6_addr, nat.ptr(la_part), m, k, nat.stream_of(x2))


def _la_reduce(la_part: Tensor) -> Tensor:
    p, m, r = (int(d) for d in la_part.shape)
    la = torch.empty(m, r, dtype=torch.bfloat16, device=la_part.device)
    nat.call("gwa_svdq_la_reduce", nat.ptr(la_part), p, m, r, nat.ptr(la), nat.stream_of(la_part))
    return la


@torch.library.custom_op("cozy_gen_worker::svdq_la_reduce", mutates_args=())
def svdq_la_reduce(la_part: Tensor) -> Tensor:
    """bf16 la [M, rank] = the fixed-order fp32 sum of the partial slots ``la_part`` [P, M, rank]."""
    name = "svdq_la_reduce"
    _check_dtype(name, la_part, torch.float32, what="la_part")
    _check_cuda(name, la_part=la_part)
    if la_part.dim() != 3 or int(la_part.shape[0]) < 1 or int(la_part.shape[2]) % 16:
        raise SvdqOpError(f"{name}: la_part must be [P >= 1, M, rank % 16 == 0], got {tuple(la_part.shape)}")
    return _la_reduce(la_part)


@svdq_la_reduce.register_fake
def _(la_part):
    return la_part.new_empty(int(la_part.shape[1]), int(la_part.shape[2]), dtype=torch.bfloat16)


@torch.library.custom_op("cozy_gen_worker::svdq_prep_proj_down_fp6", mutates_args=())
def svdq_prep_proj_down_fp6(proj_down: Tensor) -> Tensor:
    """proj_down [K, rank] bf16 -> the operand order of the fp6-lane act-quant kernel and of the next-layer
    epilogue ([K', rank], stage-major, K' = K rounded up to whole 128-row stages: a half stage's rows past K are
    zeros; K % 64 == 0). Done once per weight."""
    name = "svdq_prep_proj_down_fp6"
    _check_dtype(name, proj_down, torch.bfloat16, what="proj_down")
    _check_cuda(name, proj_down=proj_down)
    if proj_down.dim() != 2:
        raise SvdqOpError(f"{name}: proj_down must be [K, rank], got {tuple(proj_down.shape)}")
    k, r = int(proj_down.shape[0]), int(proj_down.shape[1])
    out = torch.empty(fp6_stages(k) * FP6_STAGE, r, dtype=torch.bfloat16, device=proj_down.device)
    nat.call("gwa_svdq_prep_proj_down_fp6", nat.ptr(proj_down), nat.ptr(out), k, r, nat.stream_of(proj_down))
    return out


@svdq_prep_proj_down_fp6.register_fake
def _(proj_down):
    return proj_down.new_empty(fp6_stages(int(proj_down.shape[0])) * FP6_STAGE, int(proj_down.shape[1]))


@torch.library.custom_op("cozy_gen_worker::svdq_quant_fp6", mutates_args=())
def svdq_quant_fp6(x2: Tensor, smooth: Optional[Tensor], s2: Optional[Tensor],
                   proj_down_op6: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """Kernel 1 for the fp6 lane: ``(records [K/128, M, 104], la bf16 [M, rank])`` — the codes and group scales
    as fp6 operand records (e3m2 codes + fp16 scales: the fp6 GEMM's operand format) and ``x2 @ proj_down``
    (fp32 partial sums over K ranges, reduced in a fixed order, rounded to bf16); la is [M, 0] when
    ``proj_down_op6`` (``svdq_prep_proj_down_fp6``) is None."""
    m, k = int(x2.shape[0]), int(x2.shape[-1])
    q6 = records_empty(fp6_stages(k), m, x2.device)
    r = int(proj_down_op6.shape[1]) if proj_down_op6 is not None else 0
    if not r:
        _fp6_quant_into("svdq_quant_fp6", x2, smooth, s2, None, q6, None)
        return q6, x2.new_empty(m, 0)
    name = "svdq_quant_fp6"
    if x2.dim() != 2:
        raise SvdqOpError(f"{name}: x2 must be 2-D, got {tuple(x2.shape)}")
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_dtype(name, smooth, torch.bfloat16, what="smooth")
    _check_dtype(name, proj_down_op6, torch.bfloat16, what="proj_down_op6")
    s2 = _scalar_f32(name, s2)
    _check_cuda(name, x2=x2, smooth=smooth, s2=s2, proj_down_op6=proj_down_op6)
    if k % GROUP:
        raise SvdqOpError(f"{name}: the fp6 records need K % {GROUP} == 0, got K={k}")
    if smooth is not None and smooth.numel() != k:
        raise SvdqOpError(f"{name}: smooth has {smooth.numel()} values for K={k}")
    if proj_down_op6.dim() != 2 or int(proj_down_op6.shape[0]) < fp6_stages(k) * FP6_STAGE:
        raise SvdqOpError(f"{name}: proj_down_op6 must be [>= {fp6_stages(k) * FP6_STAGE}, rank] rows in operand "
                          f"order, got {tuple(proj_down_op6.shape)}")
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    la = torch.empty(m, r, dtype=torch.bfloat16, device=x2.device)
    ws_bytes = int(nat.load().gwa_svdq_quant_fp6_la_workspace(m, k, r))
    ws = torch.empty(max(ws_bytes, 4) // 4, dtype=torch.float32, device=x2.device)
    nat.call("gwa_svdq_quant_fp6_la", nat.ptr(x2), int(x2.stride(0)), nat.ptr(smooth), nat.ptr(s2),
             nat.ptr(proj_down_op6), r, nat.ptr(q6), nat.ptr(la), nat.ptr(ws), ws_bytes, m, k, nat.stream_of(x2))
    return q6, la


@svdq_quant_fp6.register_fake
def _(x2, smooth, s2, proj_down_op6):
    m, k = int(x2.shape[0]), int(x2.shape[1])
    r = int(proj_down_op6.shape[1]) if proj_down_op6 is not None else 0
    return (x2.new_empty(fp6_stages(k), m, nat.FP6_REC, dtype=torch.uint8),
            x2.new_empty(m, r, dtype=torch.bfloat16))


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


def _epi_flags(gelu: bool, la: Optional[Tensor]) -> int:
    return (nat.EPI_GELU_TANH if gelu else 0) | (nat.EPI_LA_F32 if la is not None and la.dtype == torch.float32 else 0)


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
    _check_dtype(name, la, torch.bfloat16, torch.float32, what="la")
    _check_dtype(name, up, torch.bfloat16, what="up")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    _check_cuda(name, qa6=qa6, weight_fp6=weight_fp6, s2=s2, second=second, la=la, up=up, bias=bias)
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise SvdqOpError(f"{name}: out_dtype {out_dtype} not bf16/fp16")
    m, k = _fp6_records_k(name, qa6, "qa6")
    n, kw = _fp6_records_k(name, weight_fp6, "weight_fp6")
    if kw != k:
        raise SvdqOpError(f"{name}: activation K={k} and weight K={kw} differ")
    _check_record_slack(name, qa6, "qa6")
    _check_record_slack(name, weight_fp6, "weight_fp6")
    rank, sec_n = _epilogue_operands(name, m, n, la, up, bias, second)
    out = torch.empty(m, n, dtype=out_dtype, device=qa6.device)
    nat.call("gwa_svdq_gemm_w4a4_fp6", nat.ptr(qa6), readable_bytes(qa6), nat.ptr(weight_fp6),
             readable_bytes(weight_fp6), nat.ptr(s2), nat.ptr(second), sec_n, nat.ptr(la), nat.ptr(up), rank, nat.ptr(bias), nat.ptr(out), _dt_code(out_dtype),
             _epi_flags(gelu, la), m, n, k, nat.stream_of(qa6))
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


def linear_fp6_workspace_bytes(m: int, k: int, rank: int) -> int:
    """Workspace bytes of one ``svdq_forward_fp6`` call (activation records + slack, la partial slots, la)."""
    return int(nat.load().gwa_svdq_w4a4_linear_fp6_workspace(m, k, rank))


@torch.library.custom_op("cozy_gen_worker::svdq_forward_fp6", mutates_args=())
def svdq_forward_fp6(x2: Tensor, smooth: Optional[Tensor], s2: Optional[Tensor], proj_down_op6: Optional[Tensor],
                     weight_fp6: Tensor, second: Optional[Tensor], proj_up: Optional[Tensor], bias: Optional[Tensor],
                     out_dtype: torch.dtype, gelu: bool) -> Tensor:
    """The whole fp6-lane linear in one library call (``_SvdqFusedLinear.forward``, ``models/svdq_fused.py:516-527``):
    kernel 1 into a workspace (records, la partial slots), the fixed-order la reduction and the GEMM with its
    epilogue; bit-identical to ``svdq_quant_fp6`` followed by ``svdq_w4a4_linear_fp6``."""
    name = "svdq_forward_fp6"
    if x2.dim() != 2:
        raise SvdqOpError(f"{name}: x2 must be 2-D, got {tuple(x2.shape)}")
    s2 = _scalar_f32(name, s2)
    if second is not None and second.dtype != torch.float32:
        second = second.float().contiguous()
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_dtype(name, smooth, torch.bfloat16, what="smooth")
    _check_dtype(name, proj_down_op6, torch.bfloat16, what="proj_down_op6")
    _check_dtype(name, weight_fp6, torch.uint8, what="weight_fp6")
    _check_dtype(name, proj_up, torch.bfloat16, what="proj_up")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise SvdqOpError(f"{name}: out_dtype {out_dtype} not bf16/fp16")
    if x2.stride(1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    _check_cuda(name, smooth=smooth, s2=s2, proj_down_op6=proj_down_op6, weight_fp6=weight_fp6, second=second,
                proj_up=proj_up, bias=bias)
    if not x2.is_cuda:
        raise SvdqOpError(f"{name}: x2 is on {x2.device}; the int4/int8 path runs on the GPU only")
    m, k = int(x2.shape[0]), int(x2.shape[1])
    if k % GROUP:
        raise SvdqOpError(f"{name}: the fp6 lane needs K % {GROUP} == 0, got K={k}")
    kp = fp6_stages(k) * FP6_STAGE  # K % 128 == 64: the records end in a half stage
    n, kw = _fp6_records_k(name, weight_fp6, "weight_fp6")
    if kw != kp:
        raise SvdqOpError(f"{name}: x2 has K={k} ({kp // FP6_STAGE} stages), weight_fp6 {kw // FP6_STAGE} stages")
    if smooth is not None and smooth.numel() != k:
        raise SvdqOpError(f"{name}: smooth has {smooth.numel()} values for K={k}")
    _check_record_slack(name, weight_fp6, "weight_fp6")
    if (proj_down_op6 is None) != (proj_up is None):
        raise SvdqOpError(f"{name}: proj_down_op6 and proj_up must both be given or both be None")
    rank = 0
    if proj_up is not None:
        rank = int(proj_up.shape[1])
        if tuple(proj_up.shape) != (n, rank) or tuple(proj_down_op6.shape) != (kp, rank):
            raise SvdqOpError(f"{name}: proj_up {tuple(proj_up.shape)} / proj_down_op6 {tuple(proj_down_op6.shape)} "
                              f"do not match [N={n}, r] / [K'={kp}, r]")
    if bias is not None and bias.numel() != n:
        raise SvdqOpError(f"{name}: bias has {bias.numel()} values for N={n}")
    out = torch.empty(m, n, dtype=out_dtype, device=x2.device)
    if m == 0:
        return out
    ws = torch.empty(linear_fp6_workspace_bytes(m, k, rank), dtype=torch.uint8, device=x2.device)
    nat.call("gwa_svdq_w4a4_linear_fp6", nat.ptr(x2), int(x2.stride(0)), nat.ptr(smooth), nat.ptr(s2),
             nat.ptr(proj_down_op6), rank, nat.ptr(weight_fp6), readable_bytes(weight_fp6), nat.ptr(second),
             0 if second is None else int(second.numel()), nat.ptr(proj_up), nat.ptr(bias), nat.ptr(out),
             _dt_code(out_dtype), nat.EPI_GELU_TANH if gelu else 0, m, n, k, nat.ptr(ws), int(ws.numel()),
             nat.stream_of(x2))
    return out


@svdq_forward_fp6.register_fake
def _(x2, smooth, s2, proj_down_op6, weight_fp6, second, proj_up, bias, out_dtype, gelu):
    return x2.new_empty(int(x2.shape[0]), int(weight_fp6.shape[1]), dtype=out_dtype)


def gemv_max_m(k: int, rank: int) -> int:
    """The most tokens the small-M path (``svdq_forward_gemv``) takes at K inputs and this rank (0: none)."""
    return int(nat.load().gwa_svdq_w4a4_gemv_max_m(k, rank))


@torch.library.custom_op("cozy_gen_worker::svdq_forward_gemv", mutates_args=())
def svdq_forward_gemv(x2: Tensor, smooth: Optional[Tensor], s2: Optional[Tensor], proj_down_op6: Optional[Tensor],
                      weight: Tensor, weight_scale: Tensor, second: Optional[Tensor], proj_up: Optional[Tensor],
                      bias: Optional[Tensor], out_dtype: torch.dtype, gelu: bool) -> Tensor:
    """The whole linear for a few tokens (``_SvdqFusedLinear.forward``, ``models/svdq_fused.py:516-527``, at
    M <= ``gemv_max_m``): the int4 weight [N, K/2] and its fp16 scales streamed once by a GEMV that quantizes
    the rows with kernel 1's quantizer (bit-identical codes and scales) and sums kernel 1's la partial slots;
    the group order and epilogue of the GEMM lane (only the low-rank sum rounds differently)."""
    name = "svdq_forward_gemv"
    if x2.dim() != 2:
        raise SvdqOpError(f"{name}: x2 must be 2-D, got {tuple(x2.shape)}")
    s2 = _scalar_f32(name, s2)
    if second is not None and second.dtype != torch.float32:
        second = second.float().contiguous()
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_dtype(name, smooth, torch.bfloat16, what="smooth")
    _check_dtype(name, proj_down_op6, torch.bfloat16, what="proj_down_op6")
    _check_dtype(name, weight, torch.uint8, what="weight")
    _check_dtype(name, weight_scale, torch.float16, what="weight_scale")
    _check_dtype(name, proj_up, torch.bfloat16, what="proj_up")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise SvdqOpError(f"{name}: out_dtype {out_dtype} not bf16/fp16")
    if x2.stride(1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    _check_cuda(name, smooth=smooth, s2=s2, proj_down_op6=proj_down_op6, weight=weight, weight_scale=weight_scale,
                second=second, proj_up=proj_up, bias=bias)
    if not x2.is_cuda:
        raise SvdqOpError(f"{name}: x2 is on {x2.device}; the int4/int8 path runs on the GPU only")
    m, k = int(x2.shape[0]), int(x2.shape[1])
    if weight.dim() != 2 or int(weight.shape[1]) * 2 != k or not weight.is_contiguous():
        raise SvdqOpError(f"{name}: weight must be contiguous [N, K/2 = {k // 2}], got {tuple(weight.shape)}")
    n = int(weight.shape[0])
    if tuple(weight_scale.shape) != (n, k // 64) or not weight_scale.is_contiguous():
        raise SvdqOpError(f"{name}: weight_scale must be contiguous [N={n}, K/64={k // 64}], got "
                          f"{tuple(weight_scale.shape)}")
    if smooth is not None and smooth.numel() != k:
        raise SvdqOpError(f"{name}: smooth has {smooth.numel()} values for K={k}")
    if (proj_down_op6 is None) != (proj_up is None):
        raise SvdqOpError(f"{name}: proj_down_op6 and proj_up must both be given or both be None")
    rank = 0
    if proj_up is not None:
        rank = int(proj_up.shape[1])
        if tuple(proj_up.shape) != (n, rank) or tuple(proj_down_op6.shape) != (k, rank):
            raise SvdqOpError(f"{name}: proj_up {tuple(proj_up.shape)} / proj_down_op6 {tuple(proj_down_op6.shape)} "
                              f"do not match [N={n}, r] / [K={k}, r]")
    if bias is not None and bias.numel() != n:
        raise SvdqOpError(f"{name}: bias has {bias.numel()} values for N={n}")
    out = torch.empty(m, n, dtype=out_dtype, device=x2.device)
    if m == 0:
        return out
    ws = torch.empty(max(int(nat.load().gwa_svdq_w4a4_linear_gemv_workspace(m, k, rank)), 256), dtype=torch.uint8,
                     device=x2.device)
    nat.call("gwa_svdq_w4a4_linear_gemv", nat.ptr(x2), int(x2.stride(0)), nat.ptr(smooth), nat.ptr(s2),
             nat.ptr(proj_down_op6), rank, nat.ptr(weight), nat.ptr(weight_scale), nat.ptr(second),
             0 if second is None else int(second.numel()), nat.ptr(proj_up), nat.ptr(bias), nat.ptr(out),
             _dt_code(out_dtype), nat.EPI_GELU_TANH if gelu else 0, m, n, k, nat.ptr(ws), int(ws.numel()),
             nat.stream_of(x2))
    return out


@svdq_forward_gemv.register_fake
def _(x2, smooth, s2, proj_down_op6, weight, weight_scale, second, proj_up, bias, out_dtype, gelu):
    return x2.new_empty(int(x2.shape[0]), int(weight.shape[0]), dtype=out_dtype)


def eager_call_ok(x2: Tensor) -> bool:
    """Whether a module forward may call a bound linear (``BoundLinearFp6``) instead of the registered op: a plain
    CUDA tensor, eager mode (not under torch.compile, no Python dispatch or torch-function mode active, which the
    op would pass through) and no autograd graph to record (the op has no autograd formula)."""
    return (type(x2) is Tensor and x2.is_cuda and not torch.compiler.is_compiling()
            and not (x2.requires_grad and torch.is_grad_enabled())
            and not torch._C._is_torch_function_mode_enabled()
            and torch._C._len_torch_dispatch_stack() == 0)


class BoundLinearFp6:
    """One fp6-lane linear's resident operands bound for eager calls: the same library entry points and
    arguments as ``svdq_forward_fp6`` (and ``svdq_forward_gemv`` up to ``gemv_max_m`` tokens), so the output is
    the op's bit for bit, without the dispatcher's and the per-call operand checks' host time. The operands are
    checked once, by running both ops on a 0-row activation; a call then checks only the activation (dtype,
    device, width; rows with an unaligned stride are copied, as the op does), allocates the output and the
    workspace and enqueues on the current stream. The pointers are those of the tensors at binding: the owner
    rebinds when any of them changes (``key``), and the binding holds them (``held``)."""

    __slots__ = ("key", "held", "device", "k", "n", "rank", "out_dtype", "gemv_max_m", "_lin", "_gemv",
                 "_lin_args", "_gemv_args", "_tail", "_ws_lin", "_ws_gemv", "_ws", "_dev_index")

    def __init__(self, *, key: tuple, held: tuple, k: int, smooth: Optional[Tensor], proj_down_op6: Optional[Tensor],
                 weight: Tensor,
                 weight_scale: Tensor, weight_fp6: Tensor, second: Optional[Tensor], proj_up: Optional[Tensor],
                 bias: Optional[Tensor], out_dtype: torch.dtype, gelu: bool, gemv_max_m: int) -> None:
        n = _fp6_records_k("BoundLinearFp6", weight_fp6, "weight_fp6")[0]
        x0 = torch.empty(0, k, dtype=torch.bfloat16, device=weight_fp6.device)
        svdq_forward_fp6(x0, smooth, None, proj_down_op6, weight_fp6, second, proj_up, bias, out_dtype, gelu)
        if gemv_max_m > 0:
            svdq_forward_gemv(x0, smooth, None, proj_down_op6, weight, weight_scale, second, proj_up, bias, out_dtype,
                              gelu)
        if second is not None and second.dtype != torch.float32:
            raise SvdqOpError("BoundLinearFp6: second must be float32 (the op would convert it per call)")
        lib = nat.load()
        self.key = key
        self.held = held  # the bound pointers' tensors stay allocated while the binding exists
        self.device = weight_fp6.device
        self._dev_index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.k, self.n = k, n
        self.rank = int(proj_up.shape[1]) if proj_up is not None else 0
        self.out_dtype = out_dtype
        self.gemv_max_m = int(gemv_max_m)
        self._lin = lib.gwa_svdq_w4a4_linear_fp6
        self._gemv = lib.gwa_svdq_w4a4_linear_gemv
        self._ws_lin = lib.gwa_svdq_w4a4_linear_fp6_workspace
        self._ws_gemv = lib.gwa_svdq_w4a4_linear_gemv_workspace
        self._ws: dict = {}
        sn = 0 if second is None else int(second.numel())
        # the arguments between the activation's (pointer, row stride) and the output pointer
        self._lin_args = (nat.ptr(smooth), None, nat.ptr(proj_down_op6), self.rank, weight_fp6.data_ptr(),
                          readable_bytes(weight_fp6), nat.ptr(second), sn, nat.ptr(proj_up), nat.ptr(bias))
        self._gemv_args = (nat.ptr(smooth), None, nat.ptr(proj_down_op6), self.rank, weight.data_ptr(),
                           weight_scale.data_ptr(), nat.ptr(second), sn, nat.ptr(proj_up), nat.ptr(bias))
        self._tail = (_dt_code(out_dtype), nat.EPI_GELU_TANH if gelu else 0)

    def workspace_bytes(self, m: int, gemv: bool) -> int:
        ws = self._ws.get((m, gemv))
        if ws is None:
            ws = (max(int(self._ws_gemv(m, self.k, self.rank)), 256) if gemv
                  else int(self._ws_lin(m, self.k, self.rank)))
            if len(self._ws) < 256:
                self._ws[(m, gemv)] = ws
        return ws

    def __call__(self, x2: Tensor) -> Optional[Tensor]:
        """The linear of bf16 activations [M, K] on this device; None when ``x2`` does not fit the binding (the
        caller then takes the op, which raises the contract error)."""
        if x2.dtype != torch.bfloat16 or x2.dim() != 2 or x2.shape[1] != self.k or x2.device != self.device:
            return None
        if x2.stride(1) != 1 or x2.stride(0) % 8:
            x2 = x2.contiguous()
        m = int(x2.shape[0])
        out = torch.empty((m, self.n), dtype=self.out_dtype, device=self.device)
        if m == 0:
            return out
        gemv = m <= self.gemv_max_m
        wsn = self.workspace_bytes(m, gemv)
        ws = torch.empty(wsn, dtype=torch.uint8, device=self.device)
        stream = torch._C._cuda_getCurrentRawStream(self._dev_index)
        fn = self._gemv if gemv else self._lin
        rc = fn(x2.data_ptr(), x2.stride(0), *(self._gemv_args if gemv else self._lin_args), out.data_ptr(),
                *self._tail, m, self.n, self.k, ws.data_ptr(), wsn, stream)
        if rc != 0:
            name = "gwa_svdq_w4a4_linear_gemv" if gemv else "gwa_svdq_w4a4_linear_fp6"
            raise nat.NativeError(f"{name} failed (code {rc}): {nat.load().gwa_last_error().decode(errors='replace')}")
        return out


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


@torch.library.custom_op("cozy_gen_worker::svdq_w4a4_linear_fp6_next", mutates_args=("next_q6", "next_la_part"))
def svdq_w4a4_linear_fp6_next(qa6: Tensor, weight_fp6: Tensor, s2: Optional[Tensor], second: Optional[Tensor],
                              la: Optional[Tensor], up: Optional[Tensor], bias: Optional[Tensor], gelu: bool,
                              next_smooth: Optional[Tensor], next_proj_down_op: Optional[Tensor], next_q6: Tensor,
                              next_la_part: Optional[Tensor], stage_offset: int, write_out: bool) -> Tensor:
    """W4A4 GEMM whose epilogue also quantizes its bf16 output as the NEXT layer's input: writes that layer's
    fp6 records into stages ``stage_offset ..`` of ``next_q6`` [S, M, 104] (bit-identical to ``svdq_quant_fp6``
    on the output with ``next_smooth``) and ``output @ proj_down_next`` as one fp32 partial per column tile
    into the first ``la_partials_next(M, N)`` slots of ``next_la_part`` [P, M, r] (``svdq_la_reduce`` makes the
    next layer's la). ``next_proj_down_op`` holds the next layer's proj_down rows for these N columns in
    operand order (a row slice of its ``proj_down_op6``). Returns the bf16 output [M, N] when ``write_out``,
    else an empty [M, 0]."""
    name = "svdq_w4a4_linear_fp6_next"
    s2 = _scalar_f32(name, s2)
    if second is not None and second.dtype != torch.float32:
        second = second.float().contiguous()
    _check_dtype(name, qa6, torch.uint8, what="qa6")
    _check_dtype(name, weight_fp6, torch.uint8, what="weight_fp6")
    _check_dtype(name, la, torch.bfloat16, torch.float32, what="la")
    _check_dtype(name, up, torch.bfloat16, what="up")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    _check_dtype(name, next_smooth, torch.bfloat16, what="next_smooth")
    _check_cuda(name, qa6=qa6, weight_fp6=weight_fp6, s2=s2, second=second, la=la, up=up, bias=bias,
                next_smooth=next_smooth, next_proj_down_op=next_proj_down_op, next_q6=next_q6,
                next_la_part=next_la_part)
    m, k = _fp6_records_k(name, qa6, "qa6")
    n, kw = _fp6_records_k(name, weight_fp6, "weight_fp6")
    if kw != k:
        raise SvdqOpError(f"{name}: activation K={k} and weight K={kw} differ")
    if n % FP6_STAGE:
        raise SvdqOpError(f"{name}: N={n} is not a multiple of {FP6_STAGE} (whole stages of the next layer)")
    if next_smooth is not None and next_smooth.numel() != n:
        raise SvdqOpError(f"{name}: next_smooth has {next_smooth.numel()} values for N={n}")
    _check_record_slack(name, qa6, "qa6")
    _check_record_slack(name, weight_fp6, "weight_fp6")
    rank, sec_n = _epilogue_operands(name, m, n, la, up, bias, second)
    q6_addr = _next_records(name, next_q6, m, n, stage_offset)
    nrank = _la_part_check(name, next_la_part, next_proj_down_op, m, n, la_partials_next(m, n))
    out = torch.empty(m, n if write_out else 0, dtype=torch.bfloat16, device=qa6.device)
    nat.call("gwa_svdq_gemm_w4a4_fp6_next", nat.ptr(qa6), readable_bytes(qa6), nat.ptr(weight_fp6),
             readable_bytes(weight_fp6), nat.ptr(s2), nat.ptr(second), sec_n, nat.ptr(la), nat.ptr(up), rank, nat.ptr(bias), nat.ptr(out) if write_out else None,
             _epi_flags(gelu, la), nat.ptr(next_smooth), nat.ptr(next_proj_down_op), nrank, q6_addr,
             nat.ptr(next_la_part), m, n, k, nat.stream_of(qa6))
    return out


@svdq_w4a4_linear_fp6_next.register_fake
def _(qa6, weight_fp6, s2, second, la, up, bias, gelu, next_smooth, next_proj_down_op, next_q6, next_la_part,
      stage_offset, write_out):
    return qa6.new_empty(int(qa6.shape[1]), int(weight_fp6.shape[1]) if write_out else 0, dtype=torch.bfloat16)


@torch.library.custom_op("cozy_gen_worker::svdq_quant_fp6_into", mutates_args=("q6", "la_part"))
def svdq_quant_fp6_into(x2: Tensor, smooth: Optional[Tensor], proj_down_op6: Optional[Tensor], q6: Tensor,
                        la_part: Optional[Tensor]) -> None:
    """Kernel 1 into stages [0, K/128) of the record buffer ``q6`` [S, M, 104] and the first
    ``la_partials_quant(M, K, rank)`` slots of ``la_part`` [P, M, rank] (``proj_down_op6``: the consumer's
    operand-order proj_down rows for these K columns). With ``svdq_w4a4_linear_fp6_next`` writing the later
    stages and slots it builds the input of a layer that takes a concatenation [x2, producer output]."""
    _fp6_quant_into("svdq_quant_fp6_into", x2, smooth, None, proj_down_op6, q6, la_part)


@svdq_quant_fp6_into.register_fake
def _(x2, smooth, proj_down_op6, q6, la_part):
    return None


@torch.library.custom_op("cozy_gen_worker::svdq_pack_weight_fp6", mutates_args=())
def svdq_pack_weight_fp6(weight: Tensor, wscales: Tensor) -> Tensor:
    """Logical int4 weights [N, K/2] + fp16 group scales [N, K/64] -> fp6 operand records
    [ceil(K/128), N, 104] (any code in [-8, 7]; K % 128 == 64 ends in a half stage: zero codes and scale)."""
    name = "svdq_pack_weight_fp6"
    _check_dtype(name, weight, torch.uint8, what="weight")
    _check_dtype(name, wscales, torch.float16, what="wscales")
    _check_cuda(name, weight=weight, wscales=wscales)
    n, kh = int(weight.shape[0]), int(weight.shape[1])
    k = 2 * kh
    if k % GROUP:
        raise SvdqOpError(f"{name}: K={k} is not a multiple of {GROUP}")
    if tuple(wscales.shape) != (n, k // GROUP):
        raise SvdqOpError(f"{name}: wscales {tuple(wscales.shape)} do not match [N={n}, K/64={k // GROUP}]")
    out = records_empty(fp6_stages(k), n, weight.device)
    nat.call("gwa_svdq_pack_weight_fp6", nat.ptr(weight.contiguous()), nat.ptr(wscales.contiguous()), nat.ptr(out),
             n, k, nat.stream_of(weight))
    return out


@svdq_pack_weight_fp6.register_fake
def _(weight, wscales):
    return weight.new_empty(fp6_stages(int(weight.shape[1]) * 2), int(weight.shape[0]), nat.FP6_REC)


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
    qa6, weight_fp6 = qa6.contiguous(), weight_fp6.contiguous()
    nat.call("gwa_svdq_group_psums_fp6", nat.ptr(qa6), readable_bytes(qa6), nat.ptr(weight_fp6),
             readable_bytes(weight_fp6), nat.ptr(out), m, n, k, nat.stream_of(qa6))
    return out


@svdq_group_psums_fp6.register_fake
def _(qa6, weight_fp6):
    return qa6.new_empty(int(qa6.shape[1]), int(weight_fp6.shape[1]), int(qa6.shape[0]) * FP6_STAGE // GROUP,
                         dtype=torch.int32)


class _Fp6WeightCache:
    """fp6 records of reference-schema weights (``wq_kn`` [K/2, N] + ``ws`` [N, K/64]), one entry per weight
    tensor pair: an entry holds weak references to both tensors and their version counters, so it is used
    only while both are alive and unmodified (an in-place update or a freed-and-reused address misses)."""

    LIMIT = 256

    def __init__(self) -> None:
        import threading
        from collections import OrderedDict

        self._lock = threading.Lock()
        self._entries: "OrderedDict[tuple, tuple]" = OrderedDict()
        self.hits = self.misses = 0

    def get(self, wq_kn: Tensor, ws: Tensor) -> Tensor:
        import weakref

        key = (wq_kn.data_ptr(), ws.data_ptr(), tuple(wq_kn.shape), tuple(ws.shape), str(wq_kn.device))
        with self._lock:
            hit = self._entries.get(key)
            if hit is not None:
                wref, sref, versions, rec = hit
                if wref() is wq_kn and sref() is ws and versions == (wq_kn._version, ws._version):
                    self._entries.move_to_end(key)
                    self.hits += 1
                    return rec
        kh, n = int(wq_kn.shape[0]), int(wq_kn.shape[1])
        w_nk = torch.empty(n, kh, dtype=torch.uint8, device=wq_kn.device)
        nat.call("gwa_transpose_2d", nat.ptr(wq_kn), nat.ptr(w_nk), kh, n, 1, nat.stream_of(wq_kn))
        rec = svdq_pack_weight_fp6(w_nk, ws)
        with self._lock:
            self._entries[key] = (weakref.ref(wq_kn), weakref.ref(ws), (wq_kn._version, ws._version), rec)
            while len(self._entries) > self.LIMIT:
                self._entries.popitem(last=False)
            self.misses += 1
        return rec

    def clear(self) -> None:
        with self._lock:
            self._entries.clear()
            self.hits = self.misses = 0


_REF_WEIGHT_FP6 = _Fp6WeightCache()


def reference_gemm_weight_cache() -> _Fp6WeightCache:
    """The process's cache of fp6 weight records behind ``svdq_gemm_w4a4_lora``."""
    return _REF_WEIGHT_FP6


@torch.library.custom_op("cozy_gen_worker::svdq_gemm_w4a4_lora", mutates_args=())
def svdq_gemm_w4a4_lora(qa: Tensor, sa: Tensor, wq_kn: Tensor, ws: Tensor, s2: Tensor, second: Tensor,
                        lora_act: Tensor, up: Tensor, bias: Optional[Tensor]) -> Tensor:
    """The reference schema (``models/svdq_fused.py:379-389``): int4 nibble activations ``qa`` [M, K/2] with
    fp16 scales ``sa`` [M, K/64], the K-major weight ``wq_kn`` [K/2, N] with ``ws`` [N, K/64], bf16 out.
    It runs the fp6 lane: the activations repacked as fp6 records each call, the weight's records built once
    per weight tensor (``reference_gemm_weight_cache``); operands outside that lane's contract (or M == 0) go
    to the general lane, which raises the contract error."""
    name = "svdq_gemm_w4a4_lora"
    _check_cuda(name, wq_kn=wq_kn, qa=qa, sa=sa, ws=ws)
    _check_dtype(name, wq_kn, torch.uint8, what="wq_kn")
    _check_dtype(name, qa, torch.uint8, what="qa")
    _check_dtype(name, sa, torch.float16, what="sa")
    _check_dtype(name, ws, torch.float16, what="ws")
    kh, n = int(wq_kn.shape[0]), int(wq_kn.shape[1])
    m, k = int(qa.shape[0]), 2 * kh
    r = int(up.shape[1]) if up is not None else 0
    if (k % GROUP == 0 and r in (0, 16, 32, 64, 128) and n % 16 == 0 and m > 0
            and tuple(qa.shape) == (m, kh) and tuple(sa.shape) == (m, k // GROUP) and tuple(ws.shape) == (n, k // GROUP)):
        w6 = _REF_WEIGHT_FP6.get(wq_kn, ws)
        q6 = svdq_pack_weight_fp6(qa, sa)
        return _fp6_impl(q6, w6, s2, second, lora_act if r else None, up if r else None, bias, torch.bfloat16, False)
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
def w8a8_quant(x2: Tensor, pertensor: bool = False, static: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    """int8 activation quant in the modes of the reference's ``quantize(x2, pertensor, static)``
    (``models/w8a8.py:261-273``): ``static`` (the layer's ``input_scale`` [1, 1] fp32) is used unchanged,
    as ``sa`` [1, 1] when ``pertensor`` else expanded to [M, 1]; without it ``sa`` is ``max(amax/127, 1e-12)``
    over the whole tensor ([1, 1]) or per token ([M, 1]). Returns (q int8 [M, K], sa)."""
    name = "w8a8_quant"
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_dtype(name, static, torch.float32, what="static")
    _check_cuda(name, x2=x2, static=static)
    if static is not None and static.numel() != 1:
        raise SvdqOpError(f"{name}: static has {static.numel()} values; the input scale is one scalar")
    m, k = int(x2.shape[0]), int(x2.shape[1])
    q = torch.empty(m, k, dtype=torch.int8, device=x2.device)
    sa = torch.empty(1 if pertensor else m, 1, dtype=torch.float32, device=x2.device)
    ws = torch.empty(1, dtype=torch.int32, device=x2.device) if pertensor and static is None else None
    nat.call("gwa_w8a8_quant", nat.ptr(x2), k, nat.ptr(q), nat.ptr(sa), nat.ptr(static), int(bool(pertensor)),
             nat.ptr(ws), m, k, nat.stream_of(x2))
    return q, sa


@w8a8_quant.register_fake
def _(x2, pertensor=False, static=None):
    m, k = int(x2.shape[0]), int(x2.shape[1])
    return x2.new_empty(m, k, dtype=torch.int8), x2.new_empty(1 if pertensor else m, 1, dtype=torch.float32)


@torch.library.custom_op("cozy_gen_worker::w8a8_scaled_mm", mutates_args=())
def w8a8_scaled_mm(qa: Tensor, weight: Tensor, sa: Tensor, weight_scale: Tensor, bias: Optional[Tensor],
                   out_dtype: torch.dtype) -> Tensor:
    """``_scaled_mm(qa, weight.t(), scale_a=sa, scale_b=weight_scale.t(), bias, out_dtype)`` on int8 codes;
    ``sa`` holds one scale per row ([M, 1], rowwise) or one for the tensor ([1, 1], pertensor)."""
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
    if int(weight.shape[1]) != k or sa.numel() not in (1, m) or weight_scale.numel() != n:
        raise SvdqOpError(f"{name}: shapes qa {tuple(qa.shape)} weight {tuple(weight.shape)} sa {tuple(sa.shape)} "
                          f"weight_scale {tuple(weight_scale.shape)} disagree")
    if bias is not None and bias.numel() != n:
        raise SvdqOpError(f"{name}: bias has {bias.numel()} values for N={n}")
    out = torch.empty(m, n, dtype=out_dtype, device=qa.device)
    nat.call("gwa_w8a8_gemm", nat.ptr(qa), nat.ptr(weight), nat.ptr(sa), sa.numel(), nat.ptr(weight_scale),
             nat.ptr(bias), _dt_code(bias.dtype) if bias is not None else 0, nat.ptr(out), _dt_code(out_dtype),
             m, n, k, nat.stream_of(qa))
    return out


@w8a8_scaled_mm.register_fake
def _(qa, weight, sa, weight_scale, bias, out_dtype):
    return qa.new_empty(int(qa.shape[0]), int(weight.shape[0]), dtype=out_dtype)


class BoundLinearW8a8:
    """A W8A8 linear's resident operands bound for eager calls: ``w8a8_quant`` then ``w8a8_scaled_mm`` as the
    ops enqueue them (same entry points and arguments, so the same output bit for bit) without the dispatcher
    and the per-call operand checks. The operands are checked once by both ops on a 0-row activation; a call
    checks the activation (bf16, contiguous [M, K] on this device) and allocates the codes, the activation
    scales and the output. The owner rebinds when an operand changes (``key``); the binding holds the tensors
    whose pointers it uses (``held``)."""

    __slots__ = ("key", "held", "device", "k", "n", "pertensor", "dynamic_pt", "out_dtype", "_quant", "_gemm",
                 "_q_args", "_g_args", "_dev_index")

    def __init__(self, *, key: tuple, held: tuple, weight: Tensor, weight_scale: Tensor, bias: Optional[Tensor],
                 static: Optional[Tensor], pertensor: bool, out_dtype: torch.dtype) -> None:
        n, k = int(weight.shape[0]), int(weight.shape[1])
        x0 = torch.empty(0, k, dtype=torch.bfloat16, device=weight.device)
        q0, sa0 = w8a8_quant(x0, pertensor, static)
        w8a8_scaled_mm(q0, weight, sa0, weight_scale, bias, out_dtype)
        lib = nat.load()
        self.key, self.held = key, held
        self.device = weight.device
        self._dev_index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.k, self.n = k, n
        self.pertensor = bool(pertensor)
        self.dynamic_pt = self.pertensor and static is None   # the per-tensor amax needs a one-word workspace
        self.out_dtype = out_dtype
        self._quant = lib.gwa_w8a8_quant
        self._gemm = lib.gwa_w8a8_gemm
        self._q_args = (nat.ptr(static), int(self.pertensor))
        self._g_args = (weight.data_ptr(), weight_scale.data_ptr(), nat.ptr(bias),
                        _dt_code(bias.dtype) if bias is not None else 0)

    def __call__(self, x2: Tensor) -> Optional[Tensor]:
        """The linear of bf16 activations [M, K]; None when ``x2`` does not fit the binding (the caller then
        takes the ops, which raise the contract error)."""
        if (x2.dtype != torch.bfloat16 or x2.dim() != 2 or x2.shape[1] != self.k or x2.device != self.device
                or not x2.is_contiguous()):
            return None
        m, k, dev = int(x2.shape[0]), self.k, self.device
        q = torch.empty((m, k), dtype=torch.int8, device=dev)
        sa = torch.empty((1 if self.pertensor else m, 1), dtype=torch.float32, device=dev)
        ws = torch.empty(1, dtype=torch.int32, device=dev) if self.dynamic_pt else None
        out = torch.empty((m, self.n), dtype=self.out_dtype, device=dev)
        stream = torch._C._cuda_getCurrentRawStream(self._dev_index)
        rc = self._quant(x2.data_ptr(), k, q.data_ptr(), sa.data_ptr(), *self._q_args, nat.ptr(ws), m, k, stream)
        if rc == 0:
            w, s, b, bdt = self._g_args
            rc = self._gemm(q.data_ptr(), w, sa.data_ptr(), sa.numel(), s, b, bdt, out.data_ptr(),
                            _dt_code(self.out_dtype), m, self.n, k, stream)
        if rc != 0:
            raise nat.NativeError(f"W8A8 linear failed (code {rc}): "
                                  f"{nat.load().gwa_last_error().decode(errors='replace')}")
        return out


# ---------------------------------------------------------------------------
# AWQ W4A16 (the adaLN modulation layers)
# ---------------------------------------------------------------------------

AWQ_GEMV_MAX_M = 16   # activation rows up to which the GEMV kernel runs; above, dequant + library GEMM


def _awq_check(name: str, weight: Tensor, wscales: Tensor, wzeros: Tensor, k: Optional[int]) -> tuple[int, int]:
    _check_dtype(name, weight, torch.uint8, what="weight")
    _check_dtype(name, wscales, torch.bfloat16, what="wscales")
    _check_dtype(name, wzeros, torch.bfloat16, what="wzeros")
    n, kk = int(weight.shape[0]), 2 * int(weight.shape[1])
    if k is not None and kk != k:
        raise SvdqOpError(f"{name}: weight {tuple(weight.shape)} holds K={kk} columns, x has K={k}")
    if n % 16 or kk % 128:
        raise SvdqOpError(f"{name}: [N={n}, K={kk}] breaks the packed contract (N % 16, K % 128)")
    if tuple(wscales.shape) != (n, kk // GROUP) or tuple(wzeros.shape) != (n, kk // GROUP):
        raise SvdqOpError(f"{name}: wscales {tuple(wscales.shape)} / wzeros {tuple(wzeros.shape)} must be "
                          f"[{n}, {kk // GROUP}]")
    return n, kk


@torch.library.custom_op("cozy_gen_worker::awq_w4a16_dequant", mutates_args=())
def awq_w4a16_dequant(weight: Tensor, wscales: Tensor, wzeros: Tensor) -> Tensor:
    """bf16 [N, K] = RN_bf16(code * wscales + wzeros): the weight ``awq_w4a16_mm`` multiplies by."""
    name = "awq_w4a16_dequant"
    _check_cuda(name, weight=weight, wscales=wscales, wzeros=wzeros)
    n, k = _awq_check(name, weight, wscales, wzeros, None)
    out = torch.empty(n, k, dtype=torch.bfloat16, device=weight.device)
    nat.call("gwa_awq_w4a16_dequant", nat.ptr(weight), nat.ptr(wscales), nat.ptr(wzeros), nat.ptr(out), n, k,
             nat.stream_of(weight))
    return out


@awq_w4a16_dequant.register_fake
def _(weight, wscales, wzeros):
    return weight.new_empty(int(weight.shape[0]), 2 * int(weight.shape[1]), dtype=torch.bfloat16)


@torch.library.custom_op("cozy_gen_worker::awq_w4a16_mm", mutates_args=())
def awq_w4a16_mm(x2: Tensor, weight: Tensor, wscales: Tensor, wzeros: Tensor, bias: Optional[Tensor]) -> Tensor:
    """The reference's packed AWQ op (``models/svdq_awq_packed.py:48-115``, same name and schema):
    x2 bf16 [M, K], weight uint8 [N, K/2] (column 2j in the low nibble of byte j), wscales / wzeros bf16
    [N, K/64], bias bf16 [N] or None -> bf16 [M, N]. Up to ``AWQ_GEMV_MAX_M`` rows run the HIP GEMV
    (the weight read once per four rows); more rows dequantize the weight to bf16 once (HIP) and run a
    library GEMM on it."""
    name = "awq_w4a16_mm"
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    _check_cuda(name, x2=x2, weight=weight, wscales=wscales, wzeros=wzeros, bias=bias)
    m, k = int(x2.shape[0]), int(x2.shape[1])
    n, _ = _awq_check(name, weight, wscales, wzeros, k)
    if bias is not None and bias.numel() != n:
        raise SvdqOpError(f"{name}: bias has {bias.numel()} values for N={n}")
    if m > AWQ_GEMV_MAX_M:
        w = awq_w4a16_dequant(weight, wscales, wzeros)
        return torch.nn.functional.linear(x2, w, bias)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=x2.device)
    nat.call("gwa_awq_w4a16_mm", nat.ptr(x2), k, nat.ptr(weight), nat.ptr(wscales), nat.ptr(wzeros), nat.ptr(bias),
             nat.ptr(out), m, n, k, nat.stream_of(x2))
    return out


@awq_w4a16_mm.register_fake
def _(x2, weight, wscales, wzeros, bias):
    return x2.new_empty(int(x2.shape[0]), int(weight.shape[0]), dtype=torch.bfloat16)


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


# ---------------------------------------------------------------------------
# nvfp4 compatibility lane
# ---------------------------------------------------------------------------

NVFP4_BLOCK = 16


def nvfp4_blocked_scale_numel(rows: int, kblocks: int) -> int:
    """Element count of the blocked scale layout (``blocked_scale_numel``, models/nvfp4_quant.py:87-89)."""
    return int(nat.load().gwa_nvfp4_blocked_scale_numel(rows, kblocks))


NVFP4_MAX_PARTS = 1024   # per-workgroup maxima of the dynamic-scale pass


def _nvfp4_quant_impl(x2: Tensor, s2: Optional[Tensor], blocked: bool,
                      dequant: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """s2 None: the dynamic scale computed on the device (returned as the 4th output), else s2 itself."""
    name = "nvfp4_quant_act"
    if x2.dim() != 2:
        raise SvdqOpError(f"{name}: x2 must be 2-D, got {tuple(x2.shape)}")
    _check_dtype(name, x2, torch.bfloat16, what="x2")
    s2 = _scalar_f32(name, s2)
    if x2.stride(1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    _check_cuda(name, s2=s2)
    if not x2.is_cuda:
        raise SvdqOpError(f"{name}: x2 is on {x2.device}; the nvfp4 lane runs on the GPU only")
    m, k = int(x2.shape[0]), int(x2.shape[1])
    if k % NVFP4_BLOCK:
        raise SvdqOpError(f"{name}: K={k} is not a multiple of {NVFP4_BLOCK}")
    kb = k // NVFP4_BLOCK
    q = torch.empty(m, k // 2, dtype=torch.uint8, device=x2.device)
    if blocked:
        sc = torch.zeros(nvfp4_blocked_scale_numel(m, kb), dtype=torch.uint8, device=x2.device)
    else:
        sc = torch.empty(m, kb, dtype=torch.uint8, device=x2.device)
    xdq = torch.empty(m, k, dtype=torch.bfloat16, device=x2.device) if dequant else x2.new_empty(0, k)
    layout = nat.NVFP4_SCALES_BLOCKED if blocked else nat.NVFP4_SCALES_FLAT
    if s2 is not None:
        nat.call("gwa_nvfp4_quant_act", nat.ptr(x2), int(x2.stride(0)), nat.ptr(s2), nat.ptr(q), nat.ptr(sc),
                 layout, nat.ptr(xdq) if dequant else None, m, k, nat.stream_of(x2))
        return q, sc, xdq, s2
    s2o = torch.empty((), dtype=torch.float32, device=x2.device)
    parts = torch.empty(NVFP4_MAX_PARTS, dtype=torch.float32, device=x2.device)
    nat.call("gwa_nvfp4_quant_act_dyn", nat.ptr(x2), int(x2.stride(0)), nat.ptr(s2o), nat.ptr(parts), nat.ptr(q),
             nat.ptr(sc), layout, nat.ptr(xdq) if dequant else None, m, k, nat.stream_of(x2))
    return q, sc, xdq, s2o


@torch.library.custom_op("cozy_gen_worker::nvfp4_quant_act", mutates_args=())
def nvfp4_quant_act(x2: Tensor, s2: Tensor, blocked: bool, dequant: bool) -> tuple[Tensor, Tensor, Tensor]:
    """nvfp4 activation quantization, bit-identical to quantize_activation_torch (models/nvfp4_quant.py:92-103):
    ``(codes uint8 [M, K/2], e4m3 scale bytes (flat [M, K/16] or blocked), dequantized bf16 [M, K] or [0, K])``;
    the dequantized activations are code * scale without s2 (exact in bf16)."""
    return _nvfp4_quant_impl(x2, s2, blocked, dequant)[:3]


@nvfp4_quant_act.register_fake
def _(x2, s2, blocked, dequant):
    m, k = int(x2.shape[0]), int(x2.shape[1])
    kb = k // NVFP4_BLOCK
    sc = (x2.new_empty(((m + 127) // 128) * 128 * ((kb + 3) // 4) * 4, dtype=torch.uint8) if blocked
          else x2.new_empty(m, kb, dtype=torch.uint8))
    return (x2.new_empty(m, k // 2, dtype=torch.uint8), sc, x2.new_empty(m if dequant else 0, k))


@torch.library.custom_op("cozy_gen_worker::nvfp4_quant_act_dyn", mutates_args=())
def nvfp4_quant_act_dyn(x2: Tensor, blocked: bool, dequant: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``nvfp4_quant_act`` with the forward's dynamic second-level scale (models/w4a4.py:342-343) computed on the
    device: ``(codes, scales, dequantized bf16 or [0, K], s2 fp32 0-d)``."""
    return _nvfp4_quant_impl(x2, None, blocked, dequant)


@nvfp4_quant_act_dyn.register_fake
def _(x2, blocked, dequant):
    m, k = int(x2.shape[0]), int(x2.shape[1])
    kb = k // NVFP4_BLOCK
    sc = (x2.new_empty(((m + 127) // 128) * 128 * ((kb + 3) // 4) * 4, dtype=torch.uint8) if blocked
          else x2.new_empty(m, kb, dtype=torch.uint8))
    return (x2.new_empty(m, k // 2, dtype=torch.uint8), sc, x2.new_empty(m if dequant else 0, k),
            x2.new_empty((), dtype=torch.float32))


@torch.library.custom_op("cozy_gen_worker::quant_nvfp4_act", mutates_args=())
def quant_nvfp4_act(x2: Tensor, s2: Tensor) -> tuple[Tensor, Tensor]:
    """The reference op's contract (models/nvfp4_quant.py:185-187): (packed codes [M, K/2], e4m3 scales in the
    cuBLAS blocked layout)."""
    if s2 is None:
        raise SvdqOpError("quant_nvfp4_act: s2 is required")
    q, sc, _, _ = _nvfp4_quant_impl(x2, s2, True, False)
    return q, sc.view(torch.float8_e4m3fn)


@quant_nvfp4_act.register_fake
def _(x2, s2):
    m, k = int(x2.shape[0]), int(x2.shape[1])
    kb = k // NVFP4_BLOCK
    return (x2.new_empty(m, k // 2, dtype=torch.uint8),
            x2.new_empty(((m + 127) // 128) * 128 * ((kb + 3) // 4) * 4, dtype=torch.float8_e4m3fn))


@torch.library.custom_op("cozy_gen_worker::nvfp4_dequant", mutates_args=())
def nvfp4_dequant(q: Tensor, scales: Tensor, blocked: bool) -> Tensor:
    """codes uint8 [rows, K/2] + e4m3 scales (flat [rows, K/16] or blocked bytes) -> bf16 [rows, K] = code *
    scale, exact (dequantize_nvfp4_tensor, models/w4a4.py:157-164, without the second-level scale)."""
    name = "nvfp4_dequant"
    if scales.dtype == torch.float8_e4m3fn:
        scales = scales.view(torch.uint8)
    _check_dtype(name, q, torch.uint8, what="q")
    _check_dtype(name, scales, torch.uint8, what="scales")
    _check_cuda(name, q=q, scales=scales)
    if q.dim() != 2:
        raise SvdqOpError(f"{name}: q must be [rows, K/2], got {tuple(q.shape)}")
    rows, k = int(q.shape[0]), 2 * int(q.shape[1])
    if k % NVFP4_BLOCK:
        raise SvdqOpError(f"{name}: K={k} is not a multiple of {NVFP4_BLOCK}")
    kb = k // NVFP4_BLOCK
    need = nvfp4_blocked_scale_numel(rows, kb) if blocked else rows * kb
    if scales.numel() != need:
        raise SvdqOpError(f"{name}: {scales.numel()} scales for [{rows}, {kb}] blocks ({'blocked' if blocked else 'flat'}"
                          f" layout needs {need})")
    out = torch.empty(rows, k, dtype=torch.bfloat16, device=q.device)
    nat.call("gwa_nvfp4_dequant", nat.ptr(q), nat.ptr(scales), nat.NVFP4_SCALES_BLOCKED if blocked else
             nat.NVFP4_SCALES_FLAT, nat.ptr(out), rows, k, nat.stream_of(q))
    return out


@nvfp4_dequant.register_fake
def _(q, scales, blocked):
    return q.new_empty(int(q.shape[0]), 2 * int(q.shape[1]), dtype=torch.bfloat16)


@torch.library.custom_op("cozy_gen_worker::nvfp4_scale_bias", mutates_args=("y",))
def nvfp4_scale_bias(y: Tensor, s2: Tensor, ws2: Tensor, bias: Optional[Tensor]) -> None:
    """In place on bf16 y [M, N]: y = RN_bf16(RN_bf16(y * RN_bf16(s2 * ws2)) + bias), the nvfp4 module's
    epilogue (models/w4a4.py:349-351) in one pass."""
    name = "nvfp4_scale_bias"
    _check_dtype(name, y, torch.bfloat16, what="y")
    _check_dtype(name, bias, torch.bfloat16, what="bias")
    s2, ws2 = _scalar_f32(name, s2), _scalar_f32(name, ws2)
    _check_cuda(name, y=y, s2=s2, ws2=ws2, bias=bias)
    if y.dim() != 2 or int(y.shape[1]) % 8:
        raise SvdqOpError(f"{name}: y must be [M, N] with N % 8 == 0, got {tuple(y.shape)}")
    if bias is not None and bias.numel() != int(y.shape[1]):
        raise SvdqOpError(f"{name}: bias has {bias.numel()} values for N={int(y.shape[1])}")
    nat.call("gwa_nvfp4_scale_bias", nat.ptr(y), nat.ptr(s2), nat.ptr(ws2), nat.ptr(bias), int(y.shape[0]),
             int(y.shape[1]), nat.stream_of(y))


@nvfp4_scale_bias.register_fake
def _(y, s2, ws2, bias):
    return None
