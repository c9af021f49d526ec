"""GPU test of the full-size Flux-shaped DiT (the bench line's config: hidden 3072, 24 heads, MLP 12288,
19 dual + 38 single blocks, 4096 image + 512 text tokens, every linear W4A4 rank 32 on the int4 lane).

At this size there is no oracle chain to hold the output against (the per-linear oracle checks run at the
same shapes in tests/test_gpu_config3.py and tests/test_gpu_kernels.py), so the test holds properties of
the whole forward: finite output of the right shape, two eager forwards bit-identical (every kernel is
deterministic: fixed-order la sums, no atomics in any accumulation), a HIP-graph replay bit-identical to
eager, and agreement with the same weights run on the dense lane (each layer folded to one bf16 Linear)
within the drift that int4 activation quantization compounds over 57 blocks (cosine 0.999 measured).
Those checks run with this package's attention kernel; the model with torch's SDPA (config 4 as stated, the
bench's default DiT line) is held to a finite output, a graph replay equal to eager and agreement with it.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native

    _native.load()
    assert torch.cuda.is_available()
    yield


def _cos(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    return float(a @ b / (a.norm() * b.norm()))


def test_full_size_dit_forward():
    from gen_worker_amd.flux_dit import FluxDiT, FluxDiTConfig, inputs
    from gen_worker_amd.svdq import SvdqW4A4Linear

    cfg = FluxDiTConfig()
    args = inputs(cfg)
    m4 = FluxDiT("w4a4", cfg, device=DEV, lane="int4", attention="flash")
    assert m4.lane == "int4"
    assert sum(isinstance(m, SvdqW4A4Linear) for m in m4.modules()) > 4 * (cfg.n_dual + cfg.n_single)
    with torch.no_grad():
        y1 = m4(*args)
        y2 = m4(*args)
    torch.cuda.synchronize()
    assert tuple(y1.shape) == (cfg.img_tokens, cfg.in_channels) and y1.dtype == torch.bfloat16
    assert bool(torch.isfinite(y1).all())
    assert torch.equal(y1, y2), "two eager forwards differ"

    # one forward captured in a HIP graph, replayed twice with eager work between the replays
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            yg = m4(*args)
    torch.cuda.synchronize()
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y1), "graph replay differs from eager"
        with torch.no_grad():
            m4(*args)  # eager work between replays
        torch.cuda.synchronize()
    del g, yg

    # the dual blocks' text stream and the single blocks' MLP branch on a second HIP stream, the modulation
    # linears on a third (the bench's configuration): the same kernels on the same inputs, so the same bits,
    # eager and graph-replayed
    side = torch.cuda.Stream()
    for blk in list(m4.dual) + list(m4.single):
        blk.side = side
    m4.mod_stream = torch.cuda.Stream()  # and the modulation linears queued ahead on a third stream
    with torch.no_grad():
        y3 = m4(*args)
    torch.cuda.synchronize()
    assert torch.equal(y3, y1), "two-stream forward differs from one stream"
    g = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            yg = m4(*args)
    torch.cuda.synchronize()
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y1), "two-stream graph replay differs"
    for blk in list(m4.dual) + list(m4.single):
        blk.side = None
    m4.mod_stream = None
    del g, yg, y3

    md = FluxDiT("w4a4", cfg, device=DEV, lane="dense", attention="flash")
    assert md.lane == "dense" and not any(isinstance(m, SvdqW4A4Linear) for m in md.modules())
    with torch.no_grad():
        yd = md(*args)
    torch.cuda.synchronize()
    cos = _cos(y1, yd)
    print(f"full-size DiT: cosine(int4 lane, dense lane) = {cos:.4f}")
    assert bool(torch.isfinite(yd).all())
    assert cos > 0.99, cos


def test_full_size_dit_forward_sdpa():
    """Config 4 as stated: the same int4-lane model with torch's bf16 SDPA in every block (flash /
    memory-efficient kernels only). Finite, a HIP-graph replay equal to the eager forward, and within the
    attention kernels' difference of the model run with gwa_dit_attention."""
    from gen_worker_amd.flux_dit import ATTENTION, FluxDiT, FluxDiTConfig, inputs

    cfg = FluxDiTConfig()
    args = inputs(cfg)
    ms = FluxDiT("w4a4", cfg, device=DEV, lane="int4", attention="sdpa", streams=2)
    with torch.no_grad():
        y1 = ms(*args)
    torch.cuda.synchronize()
    assert tuple(y1.shape) == (cfg.img_tokens, cfg.in_channels) and bool(torch.isfinite(y1).all())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            yg = ms(*args)
    torch.cuda.synchronize()
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y1), "SDPA model: graph replay differs from eager"
        with torch.no_grad():
            ms(*args)
        torch.cuda.synchronize()
    del g, yg
    for blk in list(ms.dual) + list(ms.single):
        blk.attn = ATTENTION["flash"]
    with torch.no_grad():
        yf = ms(*args)
    torch.cuda.synchronize()
    cos = _cos(y1, yf)
    print(f"full-size DiT: cosine(SDPA, gwa_dit_attention) = {cos:.5f}")
    assert cos > 0.99, cos
