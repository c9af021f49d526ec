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


# BASELINE configs
C0 = dict(m=256, k=3072, n=3072, outlier_frac=0.01, outlier_scale=20.0)
C1 = dict(m=4608, k=3072, n=3072, rank=32, outlier_frac=0.005, outlier_scale=30.0)
C2 = dict(m=4608, d=3072, h=12288, rank=32, outlier_frac=0.005, outlier_scale=30.0)   # fc1 -> GELU -> fc2
C3 = dict(ms=(256, 1024, 4608, 16384), k=3072, n=9216, rank=32, outlier_frac=0.005, outlier_scale=30.0)  # QKV
