"""Benchmark of the SVDQuant W4A4 linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
    python bench.py --only {step,gemm,quant,copy,awq,w8a8,w8a8_gemm,dit} [--iters N] (profiling driver)
    python bench.py --workload {mlp,qkv,dit,mod,nvfp4,w8a8}  (configs 2-4, modulation layers, nvfp4 lane,
                                                              the int8 GEMM sweep)

A step is one pass of the hot path over one batch of synthetic input: the
config-1 SVDQuant W4A4 linear (M = 4096 image + 512 text tokens = 4608,
K = N = 3072, rank 32, group 64, bf16 in/out) on the module's fp6 lane:
kernel 1 (smoothing + int4 act-quant + x @ proj_down, codes and scales
written as fp6 operand records) then kernel 2 (W4A4 GEMM on the fp6 MFMA +
low-rank/bias epilogue). Inputs are resident in HBM before the timed region. The K timed
steps are captured once into a HIP graph and replayed, so host launch cost
is not part of the figure; the eager (per-op Python dispatch) rate is
reported beside it. The timed replay follows at least 40 ms of untimed
replays of the same graph: after an idle gap the shader clock ramps up over
the first ~20 ms of load (the first replays run up to 15 % slower). ``value`` is the linear's throughput in int-TOPS
(2*M*N*K per step).

The ``roofline`` object covers the dominant kernel (the GEMM): its average
launch duration comes from HIP events around a graph of K back-to-back GEMM
launches on the stream they run on; ``traffic`` is the HBM bytes per launch
measured with rocprofv3 FETCH_SIZE / WRITE_SIZE, scaled by the same
counters' reading for a copy of known size (profiles/w4a4_gemm_c1_traffic.json,
written by ``--summarize-traffic``).
``cpu_baseline`` times the reference's CPU serving lane (dense fold + one
bf16 Linear) on a bounded sample of the same workload, and under
``other_configs`` the CPU path of config 0 (W8A8, M=256) and of config 3's
QKV linear at M=256 and 1024. The metric's second half, the config-4 DiT step
(every linear W4A4 on the int4 lane, against the same model with bf16 GEMMs,
each forward one HIP graph replayed ``--dit-steps`` times), goes into the same
line as ``dit_step_ms`` and ``dit_bf16_step_ms``, with the arming gate's own
decision on the box as ``dit_gate_lane``. It runs first, as ``--workload dit``
in a child process started before this process touches the GPU: its own
allocator and memory state, and a failure there leaves the config-1 line
standing (``dit_error`` instead of the dit_* figures). Prints ONE JSON line on
stdout; progress goes to stderr.

``--only`` runs one piece eagerly ``--iters`` times (after 3 warmups) and
prints nothing on stdout: it is the command the committed rocprofv3
summaries under profiles/ were taken with.
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "python-gen-worker_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "W4A4 linear TOPS (% int8 MFMA peak) at M=4608 K=N=3072; DiT step ms"
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, 5.0 POP/s
TILE_NAMES = {0: "256x256", 1: "256x128", 2: "128x128", 3: "192x256", 4: "288x192", 5: "256x192"}
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
COPY_BYTES = 64 << 20        # calibration copy for the traffic counters


ATTENTION_DESC = {"sdpa": "torch bf16 scaled_dot_product_attention (flash / memory-efficient kernels only)",
                  "flash": "bf16 flash attention (gwa_dit_attention)"}
STREAMS_DESC = ("both models: dual blocks' text stream and single blocks' MLP branch on a second HIP stream, the "
                "modulation linears queued on a third")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


WARM_MS = 40.0  # untimed load before a timed replay: the shader clock ramps up over the first ~20 ms of load


def graph_time_ms(torch, fn, reps: int, warm_calls: int = 0) -> float:
    """Average ms of ``fn`` per call from ONE timed replay of a HIP graph holding ``reps`` back-to-back calls,
    synchronized on both sides and timed with events on the stream the graph runs on. Before it the graph is
    replayed untimed for at least ``warm_calls`` calls and at least WARM_MS of load (page-in, and the clock
    ramp: right after an idle gap the first ~20 ms of replays run up to 15 % slower than steady state)."""
    from gen_worker_amd.graphs import capture_graph

    def body() -> None:
        for _ in range(reps):
            fn()  # each call's outputs are released before the next one, as in eager use

    g = capture_graph(body)[0]
    cur = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    g.replay()                                   # first replay: page-in; its time sizes the warm-up
    e1.record(cur)
    torch.cuda.synchronize()
    first_ms = max(e0.elapsed_time(e1), 1e-3)
    warm = max(-(-warm_calls // reps), int(WARM_MS / first_ms) + 1)
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    e0.record(cur)
    g.replay()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _counter_median_kib(run_dir: Path, kernel_substr: str) -> tuple[str, float]:
    """Median per-dispatch value of the single counter collected in ``run_dir`` for the first kernel whose
    name contains ``kernel_substr`` (rocprofv3 ``--output-format csv``)."""
    import csv
    import statistics

    files = sorted(run_dir.rglob("*counter_collection.csv"))
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {run_dir}")
    vals: dict[str, list[float]] = {}
    for f in files:
        with f.open() as fh:
            for row in csv.DictReader(fh):
                name = row["Kernel_Name"]
                if kernel_substr in name:
                    vals.setdefault(name, []).append(float(row["Counter_Value"]))
    if not vals:
        raise KeyError(f"no kernel matching {kernel_substr!r} in {run_dir}")
    name = sorted(vals)[0]
    return name, statistics.median(vals[name])


def summarize_traffic(d: Path) -> int:
    """HBM bytes per launch of the GEMM and kernel 1 from FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each
    scaled by what the same counter reads for a copy of COPY_BYTES."""
    import torch  # noqa: F401  (only for the package's shape helpers)

    from gen_worker_amd import synthetic
    from gen_worker_amd.svdq import act_quant_bytes

    cf = _counter_median_kib(d / "f_copy", "copyBuffer")[1]
    cw = _counter_median_kib(d / "w_copy", "copyBuffer")[1]
    ff, wf = COPY_BYTES / 1024.0 / cf, COPY_BYTES / 1024.0 / cw
    cfg = synthetic.C1
    m, n, k, r = cfg["m"], cfg["n"], cfg["k"], cfg["rank"]
    gemm_alg = (m + n) * (k // 128) * 104 + m * r * 2 + n * r * 2 + n * 2 + m * n * 2
    out = {"workload": "svdq_w4a4_linear_c1 (M=4608, N=K=3072, rank 32, bf16 out)",
           "calibration": {"copy_bytes": COPY_BYTES, "copy_fetch_size_kib": cf, "copy_write_size_kib": cw,
                           "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)}}
    for key, sub, alg in (("gemm", "w4a4_gemm_fp6", gemm_alg),
                          ("act_quant", "svdq_quant_fp6_kernel", act_quant_bytes(m, k, r, fp6=True))):
        w = "gemm" if key == "gemm" else "quant"
        name, f_kib = _counter_median_kib(d / f"f_{w}", sub)
        _, w_kib = _counter_median_kib(d / f"w_{w}", sub)
        rd, wr = int(f_kib * 1024 * ff), int(w_kib * 1024 * wf)
        out[key] = {"kernel": name, "fetch_size_kib_per_launch": f_kib, "write_size_kib_per_launch": w_kib,
                    "hbm_read_bytes_per_launch": rd, "hbm_write_bytes_per_launch": wr,
                    "hbm_bytes_per_launch": rd + wr, "algorithmic_bytes_per_launch": alg}
    path = ROOT / "profiles" / "w4a4_gemm_c1_traffic.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out, indent=1))
    return 0


def dit_step_pair(steps: int, warmup: int, modulation: str = "w4a4", attention: str = "sdpa") -> dict:
    """Config 4: one Flux-dev-shaped denoiser forward (batch 1, 4096 image + 512 text tokens, 19 + 38
    blocks), every linear W4A4 rank 32 on the int4 lane (``modulation="awq"``: the one-token adaLN modulation
    linears AWQ W4A16, as an svdq checkpoint stores them) vs the same model with bf16 nn.Linear GEMMs; the
    same attention (``"sdpa"``: torch's bf16 SDPA, as config 4 states; ``"flash"``: gwa_dit_attention), block
    glue and stream overlap in both. The W4A4 model is pinned to the int4 lane (the path being measured); the
    arming gate's own decision on this box is reported beside it as ``gate_lane``. Each model's forward is
    captured once in a HIP graph and replayed ``steps`` times."""
    import gc

    import torch

    from gen_worker_amd.flux_dit import FluxDiT, FluxDiTConfig, inputs, time_step_ms

    cfg = FluxDiTConfig()
    args_in = inputs(cfg)
    res = {"cfg": cfg}
    from gen_worker_amd.qualify import resolve_lane

    res["gate_lane"] = resolve_lane()
    for kind in ("w4a4", "bf16"):
        log(f"bench: building the {kind} DiT ({attention} attention)")
        model = FluxDiT(kind, cfg, modulation=modulation, lane="int4" if kind == "w4a4" else None, streams=2,
                        attention=attention)
        res[kind + "_lane"] = model.lane
        torch.cuda.synchronize()
        log(f"bench: timing the {kind} DiT step ({steps} graph replays, {model.lane} lane)")
        res[kind] = time_step_ms(model, args_in, steps=steps, warmup=warmup)
        with torch.no_grad():
            y = model(*args_in)
        res[kind + "_finite"] = bool(torch.isfinite(y).all())
        del model, y
        gc.collect()
        torch.cuda.empty_cache()
    return res


def bench_dit(args) -> int:
    """Config 4 as its own bench line (see ``dit_step_pair``), with ``--modulation``."""
    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native
    from gen_worker_amd.flux_dit import block_int_ops

    _native.load()
    torch.cuda.set_device(0)
    res = dit_step_pair(args.steps, args.warmup, args.modulation, args.attention)
    cfg = res["cfg"]
    ops_ = block_int_ops(cfg)
    out = {"metric": "DiT step ms (Flux-dev-shaped, batch 1, 4096+512 tokens, 19+38 blocks)",
           "value": round(res["w4a4"], 3), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": False, "dtype": "int4", "data": "synthetic",
           "config": {"workload": "flux_dit_c4", "hidden": cfg.hidden, "heads": cfg.heads, "mlp": cfg.mlp,
                      "dual_blocks": cfg.n_dual, "single_blocks": cfg.n_single, "img_tokens": cfg.img_tokens,
                      "txt_tokens": cfg.txt_tokens, "rank": cfg.rank, "attention": ATTENTION_DESC[args.attention],
                      "modulation": ("W4A4 (one token)" if args.modulation == "w4a4"
                                     else "AWQ W4A16 g64 (one token)"),
                      "lane": res["w4a4_lane"], "gate_lane": res["gate_lane"],
                      "streams": STREAMS_DESC, "timing": "forward captured in one HIP graph, replayed"},
           "bf16_gemm_ms": round(res["bf16"], 3), "speedup_vs_bf16": round(res["bf16"] / res["w4a4"], 4),
           "block_linear_int_ops": ops_, "outputs_finite": {"w4a4": res["w4a4_finite"], "bf16": res["bf16_finite"]}}
    print(json.dumps(out), flush=True)
    return 0


def run_dit_child(args) -> dict:
    """The default line's DiT half: ``--workload dit`` (torch SDPA attention, config 4 as stated) with
    ``--dit-steps`` graph replays per model, in a child process whose progress goes to this stderr. Returns
    the line's dit_* keys, or ``dit_error`` when the child fails or prints no line."""
    import subprocess

    cmd = [sys.executable, "-u", str(Path(__file__).resolve()), "--workload", "dit", "--steps", str(args.dit_steps),
           "--warmup", "1", "--modulation", args.modulation, "--attention", "sdpa"]
    log("bench: the config-4 DiT pair in a child process (" + " ".join(cmd[3:]) + ")")
    try:
        res = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=900)
    except subprocess.TimeoutExpired:
        return {"dit_error": "the DiT child process ran past 900 s"}
    lines = [ln for ln in res.stdout.splitlines() if ln.startswith("{")]
    if res.returncode != 0 or not lines:
        return {"dit_error": f"the DiT child process exited with code {res.returncode}"}
    try:
        d = json.loads(lines[-1])
        return {"dit_step_ms": d["value"], "dit_bf16_step_ms": d["bf16_gemm_ms"],
                "dit_speedup_vs_bf16": d["speedup_vs_bf16"], "dit_lane": d["config"]["lane"],
                "dit_gate_lane": d["config"]["gate_lane"], "dit_modulation": args.modulation,
                "dit_attention": ATTENTION_DESC["sdpa"], "dit_streams": STREAMS_DESC,
                "dit_outputs_finite": bool(d["outputs_finite"]["w4a4"] and d["outputs_finite"]["bf16"])}
    except (ValueError, KeyError, TypeError) as e:
        return {"dit_error": f"the DiT child process printed an unreadable line ({type(e).__name__}: {e})"}


def _w4a4_module(torch, L, dev, activation=None, out_dtype=None):
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    return build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                  proj_up=L.proj_up, bias=L.bias, activation=activation, out_dtype=out_dtype,
                                  device=dev)


def bench_mlp(args) -> int:
    """Config 2: M=4608, fc1 3072 -> 12288 with GELU-tanh, fc2 12288 -> 3072, rank 32. Three variants of the
    same pair, each timed over ``--steps`` calls in one HIP graph: ``fused`` (fc2's act-quant in fc1's GEMM
    epilogue, svdq_pair_forward), ``unfused`` (the two W4A4 modules back to back: fc1's bf16 output written
    and re-quantized), ``bf16`` (two bf16 linears with torch's GELU between them)."""
    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native, synthetic
    from gen_worker_amd.svdq import svdq_pair_forward, w4a4_int_ops

    _native.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    c = synthetic.C2
    m, d, h, r = c["m"], c["d"], c["h"], c["rank"]
    log(f"bench: config-2 MLP pair M={m} {d} -> {h} -> {d} r={r}")
    L1, L2 = synthetic.w4a4_layer(h, d, r, seed_offset=0), synthetic.w4a4_layer(d, h, r, seed_offset=100)
    fc1, fc2 = _w4a4_module(torch, L1, dev, "gelu_tanh"), _w4a4_module(torch, L2, dev)
    x = synthetic.activation(m, d, outlier_frac=c["outlier_frac"], outlier_scale=c["outlier_scale"]).to(dev)
    w1, w2 = L1.w_res.to(dev, torch.bfloat16), L2.w_res.to(dev, torch.bfloat16)
    b1, b2 = L1.bias.to(dev), L2.bias.to(dev)
    F = torch.nn.functional
    variants = {
        "fused": lambda: svdq_pair_forward(x, fc1, fc2),
        "unfused": lambda: fc2(fc1(x)),
        "bf16": lambda: F.linear(F.gelu(F.linear(x, w1, b1), approximate="tanh"), w2, b2),
    }
    ops_ = 2 * w4a4_int_ops(m, h, d)
    res = {}
    for name, fn in variants.items():
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        ms = graph_time_ms(torch, fn, args.steps)
        res[name] = {"ms": round(ms, 5), "TOPS": round(ops_ / (ms * 1e-3) / 1e12, 1)}
        log(f"bench: {name}: {ms * 1e3:.1f} us  {res[name]['TOPS']} TOPS")
    out = {"metric": "MLP pair TOPS (config 2: fc1 + GELU + fc2, 2*2*M*D*H int ops)",
           "value": res["fused"]["TOPS"], "unit": "TOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": res["fused"]["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "int4", "data": "synthetic",
           "config": {"workload": "svdq_mlp_pair_c2", "M": m, "D": d, "H": h, "rank": r, "group": 64,
                      "timing": "K calls in one HIP graph replay, after >= 40 ms of untimed replays"},
           "pct_int8_peak": round(100 * res["fused"]["TOPS"] / INT8_PEAK_TOPS, 2), "variants": res,
           "speedup_fused_vs_unfused": round(res["unfused"]["ms"] / res["fused"]["ms"], 4),
           "speedup_fused_vs_bf16": round(res["bf16"]["ms"] / res["fused"]["ms"], 4)}
    print(json.dumps(out), flush=True)
    return 0


def bench_qkv(args) -> int:
    """Config 3: the QKV projection K=3072 -> N=9216 over M in {256, 1024, 4608, 16384} with bf16 and fp16
    outputs: the W4A4 module (act-quant + GEMM, rank 32), the W8A8 module (int8 act-quant + int8 GEMM) and a
    bf16 linear, each timed over ``--steps`` calls in one HIP graph."""
    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native, synthetic
    from gen_worker_amd.svdq import w4a4_int_ops
    from gen_worker_amd.w8a8 import build_int8_linear

    _native.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    c = synthetic.C3
    k, n, r = c["k"], c["n"], c["rank"]
    L = synthetic.w4a4_layer(n, k, r)
    L8 = synthetic.w8a8_layer(n, k)
    wb = L.w_res.to(dev, torch.bfloat16)
    rows = []
    for odt in (torch.bfloat16, torch.float16):
        w4 = _w4a4_module(torch, L, dev, out_dtype=odt)
        w8 = build_int8_linear(qweight=L8.qweight, weight_scale=L8.weight_scale, bias=L8.bias, compute_dtype=odt,
                               device=dev)
        wd, bd = wb.to(odt), L.bias.to(dev, odt)
        for m in c["ms"]:
            x = synthetic.activation(m, k, outlier_frac=c["outlier_frac"], outlier_scale=c["outlier_scale"]).to(dev)
            xd = x.to(odt)
            fns = {"w4a4": lambda: w4(x), "w8a8": lambda: w8(x),
                   "bf16" if odt == torch.bfloat16 else "fp16": lambda: torch.nn.functional.linear(xd, wd, bd)}
            row = {"M": m, "out_dtype": str(odt).replace("torch.", "")}
            ops_ = w4a4_int_ops(m, n, k)
            for name, fn in fns.items():
                for _ in range(args.warmup):
                    fn()
                torch.cuda.synchronize()
                ms = graph_time_ms(torch, fn, args.steps)
                row[name] = {"us": round(ms * 1e3, 2), "TOPS": round(ops_ / (ms * 1e-3) / 1e12, 1)}
            log(f"bench: qkv {row}")
            rows.append(row)
    big = next(rw for rw in rows if rw["M"] == 4608 and rw["out_dtype"] == "bfloat16")
    out = {"metric": "QKV projection TOPS (config 3: K=3072 -> N=9216; act-quant + GEMM per call)",
           "value": big["w4a4"]["TOPS"], "unit": "TOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(big["w4a4"]["us"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int4", "data": "synthetic",
           "config": {"workload": "qkv_sweep_c3", "K": k, "N": n, "rank": r, "M": list(c["ms"]),
                      "value_at": "M=4608, bf16 out, W4A4", "timing": "K calls in one HIP graph replay, after >= 40 ms of untimed replays"},
           "rows": rows}
    print(json.dumps(out), flush=True)
    return 0


def cpu_other_configs(torch, synthetic, threads: int) -> list:
    """The CPU path of the other configs BASELINE lists at CPU-runnable sizes: config 0 (W8A8, M=256,
    K=N=3072: the reference's dequant lane and the W8A8 torch chain) and config 3's QKV linear at M=256 and
    1024 (the W4A4 fallback lane), each the median of 10 after 3 warmups on this host's cores."""
    import numpy as np

    from gen_worker_amd.svdq import w4a4_int_ops
    from oracle import cpu_baseline

    b = lambda t: t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    out = []
    c0 = synthetic.C0
    L8 = synthetic.w8a8_layer(c0["n"], c0["k"])
    x0 = synthetic.activation(c0["m"], c0["k"], outlier_frac=c0["outlier_frac"], outlier_scale=c0["outlier_scale"])
    r = cpu_baseline.time_w8a8_linear_cpu(b(x0), L8.qweight.numpy(), L8.weight_scale.numpy(), L8.bias.numpy(),
                                          threads=threads)
    ops0 = w4a4_int_ops(c0["m"], c0["n"], c0["k"])
    out.append({"config": f"c0 W8A8 M={c0['m']} K=N={c0['k']}", "value": round(ops0 / r["dequant_s"] / 1e12, 4),
                "unit": "TOPS", "sample": (f"dequant lane (bf16 nn.Linear on the dequantized weight) "
                                           f"{r['dequant_s'] * 1e3:.2f} ms; W8A8 torch chain "
                                           f"{r['chain_s'] * 1e3:.2f} ms")})
    c3 = synthetic.C3
    L3 = synthetic.w4a4_layer(c3["n"], c3["k"], c3["rank"])
    for m in (256, 1024):
        x3 = synthetic.activation(m, c3["k"], outlier_frac=c3["outlier_frac"], outlier_scale=c3["outlier_scale"])
        r = cpu_baseline.time_w4a4_linear_cpu(b(x3), b(L3.smooth), L3.qweight.numpy(), L3.wscales.numpy(),
                                              b(L3.proj_down), b(L3.proj_up), b(L3.bias), threads=threads)
        out.append({"config": f"c3 QKV M={m} K={c3['k']} N={c3['n']}",
                    "value": round(w4a4_int_ops(m, c3["n"], c3["k"]) / r["fallback_s"] / 1e12, 4), "unit": "TOPS",
                    "sample": (f"fallback lane {r['fallback_s'] * 1e3:.2f} ms; oracle chain "
                               f"{r['chain_s'] * 1e3:.1f} ms")})
    return out


def bench_w8a8(args) -> int:
    """The W8A8 int8 GEMM alone (``gwa_w8a8_gemm``: per-token x per-channel scales, bf16 bias and output) at
    4096^3, the config-1 shape and config 3's QKV at 4608 and 16384 tokens, with each output tile forced and
    with the tile choice, against torch's bf16 linear on the same shape; each timed over ``--steps`` calls in
    one HIP graph."""
    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native
    from gen_worker_amd.svdq import w4a4_int_ops

    lib = _native.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cg = torch.ops.cozy_gen_worker
    g = torch.Generator(device=dev).manual_seed(3)
    rows = []
    for m, n, k in ((4096, 4096, 4096), (4608, 3072, 3072), (4608, 9216, 3072), (16384, 9216, 3072)):
        qa = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev, generator=g)
        qw = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
        sa = torch.rand(m, device=dev, generator=g) * 1e-3
        sw = torch.rand(n, device=dev, generator=g) * 1e-3
        bias = torch.randn(n, device=dev, generator=g).to(torch.bfloat16)
        xd = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
        wd = torch.randn(n, k, device=dev, generator=g).to(torch.bfloat16)
        ops_ = w4a4_int_ops(m, n, k)
        row = {"M": m, "N": n, "K": k, "tile": int(lib.gwa_w8a8_gemm_tile(m, n, k))}
        qwt = qw.t()  # torch._int_mm's [K, N] operand, column-major as hipBLASLt takes it
        variants = {"tile_128x128": 0, "tile_256x256": 1, "chosen": -1, "bf16": None, "torch_int_mm": "int_mm"}
        for name, tile in variants.items():
            if tile is None:
                fn = lambda: torch.nn.functional.linear(xd, wd, bias)  # noqa: E731
            elif tile == "int_mm":
                # the vendor library's int8 GEMM (int32 out, no epilogue), for reference only
                fn = lambda: torch._int_mm(qa, qwt)  # noqa: E731
                try:
                    fn()
                    torch.cuda.synchronize()
                except RuntimeError as e:
                    row[name] = {"unavailable": str(e).splitlines()[0][:120]}
                    continue
            else:
                lib.gwa_w8a8_gemm_force_tile(tile)
                fn = lambda: cg.w8a8_scaled_mm(qa, qw, sa, sw, bias, torch.bfloat16)  # noqa: E731
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            ms = graph_time_ms(torch, fn, args.steps)
            row[name] = {"us": round(ms * 1e3, 2), "TOPS": round(ops_ / (ms * 1e-3) / 1e12, 1)}
        lib.gwa_w8a8_gemm_force_tile(-1)
        row["vs_bf16"] = round(row["bf16"]["us"] / row["chosen"]["us"], 3)
        row["pct_int8_peak"] = round(100 * row["chosen"]["TOPS"] / INT8_PEAK_TOPS, 1)
        log(f"bench: w8a8 {row}")
        rows.append(row)
        del qa, qw, xd, wd
    big = next(rw for rw in rows if rw["M"] == 4608 and rw["N"] == 9216)
    out = {"metric": "W8A8 int8 GEMM TOPS (gwa_w8a8_gemm, per-token x per-channel scales, bf16 bias and out)",
           "value": big["chosen"]["TOPS"], "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(big["chosen"]["us"] / 1e3, 5), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
           "config": {"workload": "w8a8_gemm_sweep", "value_at": "QKV M=4608, N=9216, K=3072",
                      "timing": "K calls in one HIP graph replay, after >= 40 ms of untimed replays"},
           "roofline": {"bound": "mfma", "achieved": big["chosen"]["TOPS"], "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                        "frac": round(big["chosen"]["TOPS"] / INT8_PEAK_TOPS, 4)},
           "rows": rows}
    print(json.dumps(out), flush=True)
    return 0


def bench_mod(args) -> int:
    """The adaLN modulation linears of the config-4 DiT (one token, K=3072): the AWQ W4A16 GEMV
    (``awq_w4a16_mm``) at the dual-block (N=18432) and single-block (N=9216) shapes, M = 1 and 2, against
    the same layer as an SVDQuant W4A4 module (act-quant + GEMM) and as a bf16 linear. Each variant runs
    ``--steps`` calls in one HIP graph; the GEMV's bound is HBM (its weight, scale and zero bytes)."""
    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native, synthetic
    from gen_worker_amd.flux_dit import _awq_linear

    _native.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    k, r = 3072, 32
    rows = []
    for n in (18432, 9216):
        awq_mod = _awq_linear(k, n, 5, dev)
        L = synthetic.w4a4_layer(n, k, r)
        w4 = _w4a4_module(torch, L, dev)
        wb, bb = L.w_res.to(dev, torch.bfloat16), L.bias.to(dev, torch.bfloat16)
        for m in (1, 2):
            x = synthetic.activation(m, k, outlier_frac=0.0, outlier_scale=1.0).to(dev)
            fns = {"awq_w4a16": lambda: awq_mod(x), "w4a4": lambda: w4(x),
                   "bf16": lambda: torch.nn.functional.linear(x, wb, bb)}
            row = {"M": m, "N": n, "K": k}
            for name, fn in fns.items():
                for _ in range(args.warmup):
                    fn()
                torch.cuda.synchronize()
                row[name + "_us"] = round(graph_time_ms(torch, fn, args.steps) * 1e3, 2)
            byt = n * k // 2 + 2 * n * (k // 64) * 2 + m * k * 2 + n * 2 + m * n * 2
            row["awq_GBps"] = round(byt / row["awq_w4a16_us"] / 1e3, 1)
            row["awq_frac_hbm_peak"] = round(row["awq_GBps"] / HBM_PEAK_GBS, 4)
            log(f"bench: modulation {row}")
            rows.append(row)
    big = rows[0]
    out = {"metric": "AWQ W4A16 modulation GEMV GB/s (M=1, K=3072 -> N=18432)",
           "value": big["awq_GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(big["awq_w4a16_us"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "uint4 x bf16", "data": "synthetic",
           "config": {"workload": "awq_modulation_c4", "K": k, "N": [18432, 9216], "M": [1, 2],
                      "timing": "K calls in one HIP graph replay, after >= 40 ms of untimed replays"},
           "roofline": {"bound": "hbm", "achieved": big["awq_GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": big["awq_frac_hbm_peak"], "kernel": "awq_w4a16_gemv_kernel<1>"},
           "rows": rows}
    print(json.dumps(out), flush=True)
    return 0


def bench_nvfp4(args) -> int:
    """The nvfp4 compatibility lane at the config-1 shape (M=4608, K=N=3072): the activation quantizer
    (codes + flat scales + exact bf16 values; HBM-bound: x read, codes, scales and bf16 values written), the
    module forward (quantizer + bf16 GEMM + scale and bias) and a bf16 linear, each over ``--steps`` calls in
    one HIP graph."""
    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native, nvfp4, synthetic

    _native.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    c = synthetic.C1
    m, n, k = c["m"], c["n"], c["k"]
    g = torch.Generator().manual_seed(11)
    w = torch.randn(n, k, generator=g) * 0.02
    q, s, ws2 = nvfp4.quantize_nvfp4_tensor(w)
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    mod = nvfp4.build_nvfp4_linear(q, nvfp4.to_blocked_scales(s), ws2.reshape(1, 1), bias=bias, device=dev)
    x = synthetic.activation(m, k, outlier_frac=c["outlier_frac"], outlier_scale=c["outlier_scale"]).to(dev)
    s2 = nvfp4.dynamic_input_scale(x)
    wb = torch.ops.cozy_gen_worker.nvfp4_dequant(q.to(dev), s.view(torch.uint8).to(dev), False)
    bd = bias.to(dev)
    fns = {"quant": lambda: torch.ops.cozy_gen_worker.nvfp4_quant_act(x, s2, False, True),
           "module": lambda: mod(x),
           "bf16": lambda: torch.nn.functional.linear(x, wb, bd)}
    res = {}
    for name, fn in fns.items():
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        res[name] = graph_time_ms(torch, fn, args.steps, warm_calls=args.warmup)
    qbytes = m * k * 2 + m * k // 2 + m * k // 16 + m * k * 2
    qgbs = qbytes / (res["quant"] * 1e-3) / 1e9
    ops_ = 2 * m * n * k
    log(f"bench: nvfp4 quant {res['quant'] * 1e3:.1f} us ({qgbs:.0f} GB/s)  module {res['module'] * 1e3:.1f} us  "
        f"bf16 {res['bf16'] * 1e3:.1f} us")
    out = {"metric": "nvfp4 compatibility lane: module forward TOPS at the config-1 shape", "unit": "TOPS",
           "value": round(ops_ / (res["module"] * 1e-3) / 1e12, 1), "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(res["module"], 5), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "e2m1 x e4m3 -> bf16 products", "data": "synthetic",
           "config": {"workload": "nvfp4_linear_c1", "M": m, "N": n, "K": k, "block": 16, "s2": "dynamic",
                      "timing": "K calls in one HIP graph replay, after >= 40 ms of untimed replays"},
           "variants_us": {kk: round(v * 1e3, 2) for kk, v in res.items()},
           "roofline": {"bound": "hbm", "kernel": "nvfp4_quant_act_kernel", "achieved": round(qgbs, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(qgbs / HBM_PEAK_GBS, 4),
                        "algorithmic_bytes_per_launch": qbytes, "traffic": None}}
    print(json.dumps(out), flush=True)
    return 0


def only_awq(args) -> int:
    """``--only awq``: the dual-block modulation GEMV (M=1, K=3072 -> N=18432) eagerly ``--iters`` times
    after 3 warmups, for rocprofv3."""
    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native, synthetic
    from gen_worker_amd.flux_dit import _awq_linear

    _native.load()
    dev = torch.device("cuda:0")
    mod = _awq_linear(3072, 18432, 5, dev)
    x = synthetic.activation(1, 3072, outlier_frac=0.0, outlier_scale=1.0).to(dev)
    for _ in range(3):
        mod(x)
    torch.cuda.synchronize()
    for _ in range(args.iters):
        mod(x)
    torch.cuda.synchronize()
    log(f"bench: ran awq x{args.iters}")
    return 0


def only_dit(args) -> int:
    """``--only dit``: the config-4 W4A4 DiT (int4 lane) forward eagerly ``--iters`` times after 2 warmups,
    for rocprofv3 (each forward's kernels; the model's construction runs before them). ``--streams 1`` runs
    every kernel on one stream, so each kernel's trace duration is its own (with 2 they share the CUs)."""
    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native
    from gen_worker_amd.flux_dit import FluxDiT, FluxDiTConfig, inputs

    _native.load()
    cfg = FluxDiTConfig()
    model = FluxDiT("w4a4", cfg, modulation=args.modulation, lane="int4", streams=args.streams,
                    attention=args.attention)
    x = inputs(cfg)
    with torch.no_grad():
        for _ in range(2):
            model(*x)
        torch.cuda.synchronize()
        for i in range(args.iters):
            model(*x)
            torch.cuda.synchronize()
            log(f"bench: dit forward {i}")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-rows", type=int, default=512, help="rows of the bounded CPU sample")
    ap.add_argument("--only", choices=("step", "gemm", "quant", "copy", "awq", "w8a8", "w8a8_gemm", "dit"),
                    default=None)
    ap.add_argument("--iters", type=int, default=5)
    ap.add_argument("--streams", type=int, choices=(1, 2), default=2,
                    help="with --only dit: 1 runs the forward on one HIP stream (per-kernel profiles), 2 overlaps "
                         "the text stream, the single blocks' MLP branch and the modulation linears (the bench's)")
    ap.add_argument("--tile", type=int, default=-1,
                    help="with --only gemm/step: force the fp6 GEMM's output tile (GWA_FP6_TILE_*; -1: the model's); "
                         "with --only w8a8_gemm: the int8 GEMM's (GWA_W8A8_TILE_*)")
    ap.add_argument("--workload", choices=("c1", "mlp", "qkv", "dit", "mod", "nvfp4", "w8a8"), default="c1",
                    help="c1: the config-1 linear (the default bench line); mlp: config 2, fc1 -> GELU -> fc2 "
                         "(fused, unfused, bf16); qkv: config 3, the QKV sweep over M and output dtype (W4A4, "
                         "W8A8, bf16); dit: the config-4 Flux-shaped DiT step, W4A4 vs the same model with bf16 "
                         "GEMMs; mod: the DiT's one-token modulation linears (AWQ W4A16 GEMV vs W4A4 vs bf16); "
                         "nvfp4: the nvfp4 compatibility lane at the config-1 shape; w8a8: the int8 GEMM alone "
                         "(both tiles and the chosen one vs bf16) at 4096^3, config 1 and QKV")
    ap.add_argument("--modulation", choices=("w4a4", "awq"), default="w4a4",
                    help="the DiT's one-token adaLN modulation linears: W4A4 like every other linear (config 4 "
                         "as stated), or AWQ W4A16 as an svdq checkpoint stores them")
    ap.add_argument("--attention", choices=("sdpa", "flash"), default="sdpa",
                    help="the DiT's attention with --workload dit / --only dit: torch's bf16 SDPA (config 4 as "
                         "stated, the default line's dit_* figures) or gwa_dit_attention")
    ap.add_argument("--dit-steps", type=int, default=3,
                    help="graph replays of each DiT forward in the default (c1) line; 0 skips the DiT half")
    ap.add_argument("--summarize-traffic", metavar="DIR", default=None,
                    help="write profiles/w4a4_gemm_c1_traffic.json from the FETCH_SIZE / WRITE_SIZE runs in DIR "
                         "(subdirectories f_<w>, w_<w> for w in gemm, quant, copy)")
    args = ap.parse_args()
    if args.summarize_traffic:
        return summarize_traffic(Path(args.summarize_traffic))
    if args.only == "awq":
        return only_awq(args)
    if args.only == "dit":
        return only_dit(args)
    if args.workload != "c1":
        if args.gpus != 1:
            print("bench.py measures one GPU only", file=sys.stderr)
            return 2
        return {"dit": bench_dit, "mlp": bench_mlp, "qkv": bench_qkv, "mod": bench_mod,
                "nvfp4": bench_nvfp4, "w8a8": bench_w8a8}[args.workload](args)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build's path is a single-GPU "
              f"kernel pair; multi-GPU sharding is design-only.", file=sys.stderr)
        return 2

    # the metric's second half (the config-4 DiT pair) first, in a child process started before this process
    # touches the GPU; it has ended before the config-1 timing starts
    dit = run_dit_child(args) if args.only is None and args.dit_steps > 0 else None

    import torch

    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native, synthetic
    from gen_worker_amd.svdq import act_quant_bytes, build_svdq_w4a4_linear, w4a4_int_ops

    _native.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = synthetic.C1
    m, n, k, r = cfg["m"], cfg["n"], cfg["k"], cfg["rank"]
    log(f"bench: building config-1 layer M={m} N={n} K={k} r={r}")
    L = synthetic.w4a4_layer(n, k, r)
    x_cpu = synthetic.activation(m, k, outlier_frac=cfg["outlier_frac"], outlier_scale=cfg["outlier_scale"])
    mod = build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                 proj_up=L.proj_up, bias=L.bias, device=dev)
    x = x_cpu.to(dev)
    assert mod.lane == "fp6", "K % 128 == 0: the module must take the fp6 lane"
    ops = torch.ops.cozy_gen_worker

    def quant():
        return ops.svdq_quant_fp6(x, mod.smooth_factor, None, mod.proj_down_op6)

    qa, la = quant()

    def gemm(qa=qa, la=la):
        return ops.svdq_w4a4_linear_fp6(qa, mod.weight_fp6, None, mod.second, la, mod.proj_up, mod.bias,
                                        torch.bfloat16, False)

    def step():
        q, l = quant()
        return gemm(q, l)

    if args.only is not None:
        if args.tile >= 0 and args.only == "w8a8_gemm":
            _native.load().gwa_w8a8_gemm_force_tile(args.tile)
        elif args.tile >= 0:
            _native.load().gwa_svdq_gemm_w4a4_fp6_force_tile(args.tile)
        src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev) if args.only == "copy" else None
        dst = torch.empty_like(src) if src is not None else None
        if args.only == "w8a8_gemm":
            # the int8 GEMM alone at config 3's QKV shape (M=4608, N=9216, K=3072), the tile it chooses
            m8, n8 = m, synthetic.C3["n"]
            g8 = torch.Generator(device=dev).manual_seed(3)
            qa8 = torch.randint(-127, 128, (m8, k), dtype=torch.int8, device=dev, generator=g8)
            qw8 = torch.randint(-127, 128, (n8, k), dtype=torch.int8, device=dev, generator=g8)
            sa8, sw8 = torch.rand(m8, device=dev) * 1e-3, torch.rand(n8, device=dev) * 1e-3
            b8 = torch.randn(n8, device=dev).to(torch.bfloat16)
            cg8 = torch.ops.cozy_gen_worker
            fn = lambda: cg8.w8a8_scaled_mm(qa8, qw8, sa8, sw8, b8, torch.bfloat16)  # noqa: E731
        elif args.only == "w8a8":
            # the W8A8 linear (per-token quant + int8 GEMM) at the config-1 shape, for profiling
            from gen_worker_amd.w8a8 import build_int8_linear

            L8 = synthetic.w8a8_layer(n, k)
            lin8 = build_int8_linear(qweight=L8.qweight, weight_scale=L8.weight_scale, bias=L8.bias, device=dev)
            fn = lambda: lin8(x)  # noqa: E731
        else:
            fn = {"step": step, "gemm": gemm, "quant": quant, "copy": lambda: dst.copy_(src)}[args.only]
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        for _ in range(args.iters):
            fn()
        torch.cuda.synchronize()
        log(f"bench: ran {args.only} x{args.iters}")
        return 0

    log(f"bench: warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K steps captured in one graph, one replay, synchronize on both sides
    log(f"bench: timing {args.steps} steps (graph)")
    step_ms = graph_time_ms(torch, step, args.steps, warm_calls=args.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    gemm_ms = graph_time_ms(torch, gemm, args.steps, warm_calls=args.warmup)
    quant_ms = graph_time_ms(torch, quant, args.steps, warm_calls=args.warmup)

    int_ops = w4a4_int_ops(m, n, k)
    tile = _native.load().gwa_svdq_gemm_w4a4_fp6_tile(m, n)
    gemm_kernel = "w4a4_gemm_fp6_pipe_kernel" if tile in (4, 5) else "w4a4_gemm_fp6_kernel"
    value_tops = int_ops / (step_ms * 1e-3) / 1e12
    gemm_tops = int_ops / (gemm_ms * 1e-3) / 1e12
    qbytes = act_quant_bytes(m, k, r, fp6=True)
    qmin = act_quant_bytes(m, k, r, fp6=False)
    quant_gbs = qbytes / (quant_ms * 1e-3) / 1e9
    log(f"bench: step {step_ms * 1e3:.1f} us (eager {eager_ms * 1e3:.1f} us)  quant {quant_ms * 1e3:.1f} us "
        f"({quant_gbs:.0f} GB/s)  gemm {gemm_ms * 1e3:.1f} us ({gemm_tops:.0f} TOPS, "
        f"{100 * gemm_tops / INT8_PEAK_TOPS:.1f}% int8 peak)")

    traffic = None
    tpath = ROOT / "profiles" / "w4a4_gemm_c1_traffic.json"
    if tpath.exists():
        try:
            traffic = json.loads(tpath.read_text())["gemm"]["hbm_bytes_per_launch"]
        except (OSError, ValueError, KeyError):
            traffic = None

    cpu = None
    if not args.no_cpu:
        import numpy as np

        from oracle import cpu_baseline

        rows = max(1, min(args.cpu_rows, m))
        b = lambda t: t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
        log(f"bench: cpu baseline on {rows} rows")
        res = cpu_baseline.time_w4a4_linear_cpu(b(x_cpu[:rows]), b(L.smooth), L.qweight.numpy(), L.wscales.numpy(),
                                                b(L.proj_down), b(L.proj_up), b(L.bias))
        cpu_tops = w4a4_int_ops(rows, n, k) / res["fallback_s"] / 1e12
        cpu = {"value": round(cpu_tops, 4), "unit": "TOPS", "cores": res["threads"], "kind": "port",
               "sample": (f"reference CPU fallback lane (fold_to_dense + one bf16 nn.Linear, "
                          f"svdq_native.py:200-221) on {rows} of {m} config-1 rows, K=N={k}: median of 10 = "
                          f"{res['fallback_s'] * 1e3:.2f} ms; oracle chain (int4 act-quant -> dequant -> fp32 "
                          f"matmul) {res['chain_s'] * 1e3:.1f} ms; torch threads={res['threads']}")}
        cpu["other_configs"] = cpu_other_configs(torch, synthetic, res["threads"])

    out = {
        "metric": METRIC,
        "value": round(value_tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4",
        "data": "synthetic",
        "config": {"workload": "svdq_w4a4_linear_c1", "M": m, "N": n, "K": k, "rank": r, "group": 64,
                   "in_dtype": "bf16", "out_dtype": "bf16", "parallelism": "none",
                   "timing": "K steps in one HIP graph replay, after >= 40 ms of untimed replays"},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                     "frac": round(gemm_tops / INT8_PEAK_TOPS, 4), "traffic": traffic,
                     "kernel": gemm_kernel, "tile": TILE_NAMES.get(tile, str(tile)),
                     "algorithmic_ops_per_launch": int_ops, "avg_launch_us": round(gemm_ms * 1e3, 2)},
        "pct_int8_peak": round(100 * value_tops / INT8_PEAK_TOPS, 2),
        "eager_ms_per_step": round(eager_ms, 5),
        "act_quant": {"kernel": "svdq_quant_fp6_kernel + la_reduce_kernel", "avg_launch_us": round(quant_ms * 1e3, 2),
                      "algorithmic_bytes": qbytes, "achieved_GBps": round(quant_gbs, 1),
                      "frac_hbm_peak": round(quant_gbs / HBM_PEAK_GBS, 4),
                      # the int4 contract's minimum (nibble codes + fp16 scales + bf16 la): 36.33 MB at config 1
                      "min_bytes_int4_contract": qmin,
                      "achieved_GBps_vs_int4_min": round(qmin / (quant_ms * 1e-3) / 1e9, 1)},
        "cpu_baseline": cpu,
    }
    if dit is not None:
        out.update(dit)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
