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
