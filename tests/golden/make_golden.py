"""Generate the small golden fixtures under tests/golden/ from the CPU oracle.

The reference has no numeric fixtures for this path (its lane is nvfp4; int4
is refused at src/gen_worker/models/svdq.py:30-37), so the fixtures come from
the oracle after tests/test_oracle.py pins it. Inputs are seeded and follow
the benchmark configs' distributions at small shapes (ragged M included).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import svdq_oracle as O  # noqa: E402


def _bf16(a: np.ndarray) -> np.ndarray:
    return O.f32_to_bf16_bits(np.asarray(a, np.float32))


def _act(rng, m, k, frac, scale):
    x = rng.standard_normal((m, k)).astype(np.float32)
    n_out = int(frac * k)
    if n_out:
        x[:, rng.permutation(k)[:n_out]] *= scale
    return _bf16(x)


def make(path: Path = HERE) -> list[Path]:
    out = []
    rng = np.random.default_rng(20251201)

    # kernel 1 with smoothing + low-rank (ragged M)
    m, k, r = 77, 384, 32
    x = _act(rng, m, k, 0.02, 30.0)
    sm = _bf16(np.exp(rng.uniform(np.log(0.25), np.log(4.0), k)))
    down = _bf16(rng.standard_normal((k, r)) * 0.02)
    q, s = O.quantize_act_int4(x, sm)
    la = O.lowrank_down(x, down)
    p = path / "act_quant_m77_k384_r32.npz"
    np.savez_compressed(p, x=x, smooth=sm, proj_down=down, q=q, scales=s.view(np.uint16), la=la)
    out.append(p)

    # kernel 1 without smoothing / low-rank, second-level scale s2 = 0.75
    m, k = 33, 256
    x = _act(rng, m, k, 0.0, 1.0)
    q, s = O.quantize_act_int4(x, None, s2=0.75)
    p = path / "act_quant_m33_k256_s2.npz"
    np.savez_compressed(p, x=x, s2=np.float32(0.75), q=q, scales=s.view(np.uint16))
    out.append(p)

    # group partial sums
    qa = rng.integers(0, 256, size=(40, 96), dtype=np.uint8)
    qw = rng.integers(0, 256, size=(48, 96), dtype=np.uint8)
    p = path / "psums_m40_n48_k192.npz"
    np.savez_compressed(p, qa=qa, qw=qw, psums=O.group_psums(qa, qw))
    out.append(p)

    # full W4A4 linear
    m, n, k, r = 64, 128, 256, 16
    x = _act(rng, m, k, 0.02, 30.0)
    sm = _bf16(np.exp(rng.uniform(np.log(0.25), np.log(4.0), k)))
    qw, sw = O.quantize_weight_int4(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
    down = _bf16(rng.standard_normal((k, r)) * 0.02)
    up = _bf16(rng.standard_normal((n, r)) * 0.02)
    b = _bf16(rng.standard_normal(n) * 0.02)
    y = O.w4a4_linear(x, sm, qw, sw, down, up, b)
    qa, sa = O.quantize_act_int4(x, sm)
    p = path / "w4a4_m64_n128_k256_r16.npz"
    np.savez_compressed(p, x=x, smooth=sm, qweight=qw, wscales=sw.view(np.uint16), proj_down=down, proj_up=up,
                        bias=b, y=y, qa=qa, sa=sa.view(np.uint16))
    out.append(p)

    # W8A8 linear
    m, n, k = 33, 64, 256
    x = _act(rng, m, k, 0.01, 20.0)
    qw8, sw8 = O.quantize_weight_int8(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
    b8 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    qa8, sa8 = O.quantize_act_int8(x)
    y8 = O.w8a8_linear(x, qw8, sw8, b8)
    p = path / "w8a8_m33_n64_k256.npz"
    np.savez_compressed(p, x=x, qweight=qw8, weight_scale=sw8, bias=b8, qa=qa8, sa=sa8, y=y8)
    out.append(p)
    return out


if __name__ == "__main__":
    for p in make():
        print(p.name, p.stat().st_size)
