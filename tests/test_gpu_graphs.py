"""HIP-graph replay of the hot-path modules (how bench.py times them and how a serving loop runs them): each
module's forward captured once and replayed several times, with eager work and synchronizations between the
replays, every replay bit-identical to the eager forward on the same input."""

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
    yield


def _replays_match(fn, x, replays=3):
    with torch.no_grad():
        want = fn(x).clone()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            fn(x)   # warm the caching allocator on the capture stream
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                out = fn(x)
        torch.cuda.synchronize()
        for i in range(replays):
            noise = torch.randn(1024, 1024, device=DEV) @ torch.randn(1024, 1024, device=DEV)  # eager work between
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want), f"replay {i} differs from the eager forward"
            del noise


@pytest.mark.parametrize("m", [4608, 256, 1024])
def test_w4a4_module_graph_replays(m):
    """Kernel 1 + la reduce + the fp6 GEMM (the 256 x 256, 128 x 128 and 192 x 256 tiles by M)."""
    from gen_worker_amd import synthetic
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    n, k, r = (3072, 3072, 32) if m == 4608 else (9216, 3072, 32)
    L = synthetic.w4a4_layer(n, k, r)
    mod = build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                 proj_up=L.proj_up, bias=L.bias, device=DEV)
    x = synthetic.activation(m, k, outlier_frac=0.005, outlier_scale=30.0).to(DEV)
    print(f"graph replay: W4A4 module M={m} N={n} K={k}", flush=True)
    _replays_match(mod, x)


def test_nvfp4_module_graph_replays():
    """The nvfp4 lane with the dynamic second-level scale computed on the device."""
    from gen_worker_amd import nvfp4

    g = torch.Generator().manual_seed(2)
    w = torch.randn(1536, 1024, generator=g) * 0.02
    q, s, ws2 = nvfp4.quantize_nvfp4_tensor(w)
    mod = nvfp4.build_nvfp4_linear(q, nvfp4.to_blocked_scales(s), ws2.reshape(1, 1),
                                   bias=(torch.randn(1536, generator=g) * 0.02).to(torch.bfloat16), device=DEV)
    x = torch.randn(300, 1024, generator=g).to(torch.bfloat16).to(DEV)
    _replays_match(mod, x)


def test_awq_module_graph_replays():
    from gen_worker_amd.flux_dit import _awq_linear

    mod = _awq_linear(3072, 18432, 5, torch.device(DEV))
    x = torch.randn(1, 3072, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    _replays_match(mod, x)
