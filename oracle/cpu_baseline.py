"""CPU baseline timing of the reference's CPU path (test/bench infrastructure only).

What the reference serves for an SVDQuant linear on a host without the
kernels is the dense fallback lane: fold the dequantized weight, the
smoothing and the low-rank branch into one dense weight and run ONE bf16
``nn.Linear`` (``src/gen_worker/models/svdq_native.py:200-221``). This module
restates that lane (fold via the oracle, then ``torch.nn.functional.linear``
in bf16 on the CPU) and times it with the reference's micro-benchmark
protocol (3 warmups, median of >= 10 runs, ``models/w4a4.py:216-232``), plus
the oracle chain (act-quant -> dequant -> fp32 matmul) for comparison.
Only ``bench.py``'s ``cpu_baseline`` leg calls it.
"""

from __future__ import annotations

import os
import statistics
import time

import numpy as np
import torch

from . import svdq_oracle as O


def _median_s(fn, warmup: int = 3, iters: int = 10) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def time_w4a4_linear_cpu(x_bits: np.ndarray, smooth_bits, qw, sw, down_bits, up_bits, bias_bits,
                         threads: int | None = None, iters: int = 10) -> dict:
    """Time the fallback lane and the oracle chain on ``x_bits`` [m, K]; returns seconds and core count."""
    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    w = O.fold_to_dense(qw, sw, smooth_bits, down_bits, up_bits)
    wt = torch.from_numpy(w.astype(np.float32)).to(torch.bfloat16)
    bt = torch.from_numpy(O.bf16_bits_to_f32(bias_bits)).to(torch.bfloat16) if bias_bits is not None else None
    xt = torch.from_numpy(O.bf16_bits_to_f32(x_bits)).to(torch.bfloat16)

    def fallback():
        return torch.nn.functional.linear(xt, wt, bt)

    wd = torch.from_numpy(O.dequantize_int4(qw, sw).astype(np.float32))
    upt = torch.from_numpy(O.bf16_bits_to_f32(up_bits)) if up_bits is not None else None
    dnt = torch.from_numpy(O.bf16_bits_to_f32(down_bits)) if down_bits is not None else None
    bft = torch.from_numpy(O.bf16_bits_to_f32(bias_bits)) if bias_bits is not None else None

    def chain():
        qa, sa = O.quantize_act_int4(x_bits, smooth_bits)
        xd = torch.from_numpy(O.dequantize_int4(qa, sa).astype(np.float32))
        y = xd @ wd.t()
        if upt is not None:
            y = y + (torch.from_numpy(O.bf16_bits_to_f32(x_bits)) @ dnt) @ upt.t()
        if bft is not None:
            y = y + bft
        return y

    t_fb = _median_s(fallback, iters=iters)
    t_chain = _median_s(chain, warmup=1, iters=max(3, iters // 3))
    return {"fallback_s": t_fb, "chain_s": t_chain, "threads": threads}


def time_w8a8_linear_cpu(x_bits: np.ndarray, qw: np.ndarray, sw: np.ndarray, bias: np.ndarray | None,
                         threads: int | None = None, iters: int = 10) -> dict:
    """Config 0 on the CPU: the reference's W8A8 dequant lane (the weight dequantized once to bf16, then one
    bf16 ``nn.Linear``: the ``bf16-resident`` mode of ``models/w8a8.py:455-548``) and the W8A8 torch chain
    (per-token int8 activation quant, then the int-valued product in fp32 times the two scales, plus bias)."""
    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    wd = torch.from_numpy((qw.astype(np.float32) * sw.astype(np.float32).reshape(-1, 1))).to(torch.bfloat16)
    bt = torch.from_numpy(bias.astype(np.float32)) if bias is not None else None
    xt = torch.from_numpy(O.bf16_bits_to_f32(x_bits)).to(torch.bfloat16)
    qwt = torch.from_numpy(qw.astype(np.float32))
    swt = torch.from_numpy(sw.astype(np.float32).reshape(1, -1))

    def dequant_lane():
        return torch.nn.functional.linear(xt, wd, None if bt is None else bt.to(torch.bfloat16))

    def chain():
        x32 = xt.float()
        sa = (x32.abs().amax(dim=1, keepdim=True) / 127.0).clamp(min=1e-12)
        q = (x32 / sa).round().clamp(-127, 127)
        y = (q @ qwt.t()) * sa * swt
        return y + bt if bt is not None else y

    t_dq = _median_s(dequant_lane, iters=iters)
    t_chain = _median_s(chain, iters=iters)
    return {"dequant_s": t_dq, "chain_s": t_chain, "threads": threads}

