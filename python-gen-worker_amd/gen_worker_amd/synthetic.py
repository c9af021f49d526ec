"""Seeded synthetic inputs in the shapes and distributions of the benchmark configs.

Everything is drawn on the CPU from ``torch.Generator`` with one fixed seed
per tensor role (x=0, W=1, outlier channels=2, smooth=3, L1=4, L2=5, bias=6)
and moved afterwards, so the same call gives the same bytes on any machine.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

SEED_X, SEED_W, SEED_OUTLIER, SEED_SMOOTH, SEED_L1, SEED_L2, SEED_BIAS = 0, 1, 2, 3, 4, 5, 6


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def activation(m: int, k: int, *, outlier_frac: float, outlier_scale: float, seed: int = SEED_X,
               outlier_seed: int = SEED_OUTLIER) -> Tensor:
    """bf16 [m, k] ~ N(0, 1) with ``floor(outlier_frac * k)`` channels scaled by ``outlier_scale``."""
    x = torch.randn(m, k, generator=_gen(seed))
    n_out = int(math.floor(outlier_frac * k))
    if n_out:
        ch = torch.randperm(k, generator=_gen(outlier_seed))[:n_out]
        x[:, ch] *= outlier_scale
    return x.to(torch.bfloat16)


def smooth_factor(k: int, seed: int = SEED_SMOOTH) -> Tensor:
    """bf16 [k], log-uniform in [0.25, 4]."""
    u = torch.rand(k, generator=_gen(seed))
    return torch.exp(math.log(0.25) + u * (math.log(4.0) - math.log(0.25))).to(torch.bfloat16)


def normal(shape: tuple[int, ...], std: float, seed: int, dtype: torch.dtype = torch.float32) -> Tensor:
    return (torch.randn(*shape, generator=_gen(seed)) * std).to(dtype)


@dataclass
class W4A4Layer:
    """Logical tensors of one synthetic SVDQuant W4A4 layer."""
    w_res: Tensor            # fp32 [N, K] residual weight (quantized to int4 g64)
    qweight: Tensor          # uint8 [N, K/2]
    wscales: Tensor          # fp16 [N, K/64]
    smooth: Optional[Tensor]  # bf16 [K]
    proj_down: Optional[Tensor]  # bf16 [K, r] (L1)
    proj_up: Optional[Tensor]    # bf16 [N, r] (L2^T)
    bias: Optional[Tensor]       # bf16 [N]


def w4a4_layer(n: int, k: int, rank: int, *, smooth: bool = True, bias: bool = True, std: float = 0.02,
               seed_offset: int = 0) -> W4A4Layer:
    """Config-1 style layer: W_res ~ N(0, std) -> int4 g64; L1 [k, r], L2 [r, n] ~ N(0, std) bf16; bias ~ N(0, std)."""
    from .svdq import quantize_weight_int4

    so = seed_offset
    w = normal((n, k), std, SEED_W + so)
    qw, ws = quantize_weight_int4(w)
    sm = smooth_factor(k, SEED_SMOOTH + so) if smooth else None
    down = normal((k, rank), std, SEED_L1 + so, torch.bfloat16) if rank else None
    up = normal((rank, n), std, SEED_L2 + so, torch.bfloat16).t().contiguous() if rank else None
    b = normal((n,), std, SEED_BIAS + so, torch.bfloat16) if bias else None
    return W4A4Layer(w, qw, ws, sm, down, up, b)


@dataclass
class W8A8Layer:
    w: Tensor               # fp32 [N, K]
    qweight: Tensor         # int8 [N, K]
    weight_scale: Tensor    # fp32 [N, 1]
    bias: Optional[Tensor]  # fp32 [N]


def w8a8_layer(n: int, k: int, *, bias: bool = True, std: float = 0.02, seed_offset: int = 0) -> W8A8Layer:
    """Config-0 style layer: W ~ N(0, std) -> per-channel int8; fp32 bias ~ N(0, std)."""
    from .w8a8 import quantize_weight_int8

    w = normal((n, k), std, SEED_W + seed_offset)
    q, s = quantize_weight_int8(w)
    b = normal((n,), std, SEED_BIAS + seed_offset) if bias else None
    return W8A8Layer(w, q, s, b)


@dataclass
class SvdqFp4Layer:
    """One synthetic linear in nunchaku's svdq fp4 packaging: ``stored`` holds the file's tensors, ``w`` the
    fp32 [N, K] weight they approximate and ``bias`` the bf16 bias."""
    stored: dict
    w: Tensor
    bias: Optional[Tensor]


def svdq_fp4_layer(n: int, k: int, rank: int, *, per_channel: bool = True, smooth: bool = True,
                   bias: bool = True, std: float = 0.02, seed_offset: int = 0) -> SvdqFp4Layer:
    """An exporter's output for the weight W = (R + up @ down) / s: residual R ~ N(0, std) [N, K], low-rank
    factors up ~ N(0, std) [N, rank] and down ~ N(0, rank^-1/2) [rank, K] (bf16; the branch is as large as the
    residual, as SVDQuant's is), smoothing s. The file stores proj_down = down / s (the exporter bakes the
    smoothing in), the second scale bf16(max|R| / (6 * 448)) per row or per tensor, e4m3 block scales
    clamp(max|R_block| / (6 * second), 2^-9, 448) and the e2m1 codes of R / (scale * second), every tensor
    packed as the file stores it; ``w`` is W in fp32."""
    from .nvfp4 import _cast_e2m1
    from .svdq_checkpoint import pack_lowrank, pack_qweight, pack_vector
    from .svdq_fp4 import BLOCK, pack_micro_scales

    so = seed_offset
    resid = normal((n, k), std, SEED_W + so)
    s = smooth_factor(k, SEED_SMOOTH + so) if smooth else torch.ones(k, dtype=torch.bfloat16)
    w = resid.clone()
    stored: dict = {}
    if rank:
        down = normal((rank, k), rank ** -0.5, SEED_L1 + so, torch.bfloat16)
        up = normal((n, rank), std, SEED_L2 + so, torch.bfloat16)
        w = w + up.float() @ down.float()
        stored["proj_down"] = pack_lowrank((down.float() / s.float().reshape(1, -1)).to(torch.bfloat16).t()
                                           .contiguous(), down=True)
        stored["proj_up"] = pack_lowrank(up, down=False)
    w = w / s.float().reshape(1, -1)
    amax = resid.abs().amax(dim=1, keepdim=True) if per_channel else resid.abs().amax().reshape(1, 1)
    second = (amax / (6.0 * 448.0)).clamp(min=1e-8).to(torch.bfloat16).float()
    blocks = resid.reshape(n, k // BLOCK, BLOCK)
    bs = (blocks.abs().amax(dim=-1) / (6.0 * second)).clamp(2.0 ** -9, 448.0).to(torch.float8_e4m3fn)
    codes = _cast_e2m1((blocks / (bs.float().unsqueeze(-1) * second.unsqueeze(-1))).reshape(n, k))
    stored["qweight"] = pack_qweight(codes)
    stored["wscales"] = pack_micro_scales(bs)
    if per_channel:
        stored["wcscales"] = pack_vector(second.reshape(-1).to(torch.bfloat16), n)
    else:
        stored["wtscale"] = second.reshape(1).to(torch.bfloat16)
    if smooth:
        stored["smooth_factor"] = pack_vector(s, k)
    b = normal((n,), std, SEED_BIAS + so, torch.bfloat16) if bias else None
    if b is not None:
        stored["bias"] = pack_vector(b, n)
    return SvdqFp4Layer(stored, w, b)


# BASELINE configs
C0 = dict(m=256, k=3072, n=3072, outlier_frac=0.01, outlier_scale=20.0)
C1 = dict(m=4608, k=3072, n=3072, rank=32, outlier_frac=0.005, outlier_scale=30.0)
C2 = dict(m=4608, d=3072, h=12288, rank=32, outlier_frac=0.005, outlier_scale=30.0)   # fc1 -> GELU -> fc2
C3 = dict(ms=(256, 1024, 4608, 16384), k=3072, n=9216, rank=32, outlier_frac=0.005, outlier_scale=30.0)  # QKV
