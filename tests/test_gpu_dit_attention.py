"""The DiT's attention kernel (``gwa_dit_attention`` / ``flux_dit.attention``) against softmax attention
computed in float32 (q k^T, a float32 softmax, p v; torch matmuls on float32 operands), with torch's own
bf16 ``scaled_dot_product_attention`` measured against the same reference as the yardstick: both round the
probabilities (or their products) to bf16 on the way into p v, so the kernel must stay within a small
factor of SDPA's error, element by element and on average. Shapes: the full-size DiT's joint sequence
(4608 tokens, 24 heads; four heads against the reference), the small DiT's (256 tokens), a query count
that is not a multiple of the 128-query tile, and v as a column slice of a fused qkv output (token
stride 3 * hidden), key counts that end in a partial 64-key tile (the rows past the last key are masked)."""

from __future__ import annotations

import math

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


def _reference(q, k, v, heads):
    """float32 attention of the given heads: [S, len(heads), 128]."""
    out = []
    for h in heads:
        qh, kh, vh = q[:, h].float(), k[:, h].float(), v[:, h].float()
        p = torch.softmax((qh @ kh.t().contiguous()) / math.sqrt(qh.shape[-1]), dim=-1)
        out.append(p @ vh)
    return torch.stack(out, dim=1)


def _inputs(s, skv, heads, seed, fused_v=False):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = (torch.randn(s, heads, 128, generator=g, device=DEV) * 1.5).to(torch.bfloat16)
    k = (torch.randn(skv, heads, 128, generator=g, device=DEV) * 1.5).to(torch.bfloat16)
    if fused_v:
        qkv = torch.randn(skv, 3 * heads * 128, generator=g, device=DEV).to(torch.bfloat16)
        v = qkv[:, 2 * heads * 128:].reshape(skv, heads, 128)
    else:
        v = torch.randn(skv, heads, 128, generator=g, device=DEV).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("s,skv,heads,check,fused_v", [(4608, 4608, 24, (0, 7, 13, 23), True),
                                                       (256, 256, 4, (0, 1, 2, 3), False),
                                                       (200, 320, 3, (0, 1, 2), False),
                                                       (130, 257, 2, (0, 1), False), (96, 200, 2, (0, 1), False),
                                                       (64, 40, 2, (0, 1), True)])
def test_attention_matches_fp32_reference(s, skv, heads, check, fused_v):
    from gen_worker_amd.flux_dit import _sdpa, attention

    q, k, v = _inputs(s, skv, heads, seed=s + heads, fused_v=fused_v)
    o = attention(q, k, v).reshape(s, heads, 128)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all())
    ref = _reference(q, k, v, check)
    got = o[:, list(check)].float()
    err = (got - ref).abs()
    scale = ref.abs().max().item()
    mine = (err.max().item() / scale, err.mean().item() / ref.abs().mean().item())
    if s == skv:
        sd = _sdpa(q, k, v).reshape(s, heads, 128)[:, list(check)].float()
        e2 = (sd - ref).abs()
        theirs = (e2.max().item() / scale, e2.mean().item() / ref.abs().mean().item())
    else:
        theirs = (None, None)
    print(f"attention {s}x{skv} h{heads}: max err {mine[0]:.2e} mean rel {mine[1]:.2e}; sdpa {theirs}")
    assert mine[0] < 2e-2 and mine[1] < 5e-3, mine
    if theirs[0] is not None:
        assert mine[0] <= 3 * theirs[0] + 1e-3 and mine[1] <= 3 * theirs[1] + 1e-4, (mine, theirs)


def test_attention_deterministic_and_graph_replays():
    from gen_worker_amd.flux_dit import attention

    q, k, v = _inputs(512, 512, 8, seed=3)
    o1 = attention(q, k, v)
    o2 = attention(q, k, v)
    assert torch.equal(o1, o2)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            og = attention(q, k, v)
    torch.cuda.synchronize()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(og, o1)
        attention(q, k, v)
        torch.cuda.synchronize()


def test_attention_refuses_bad_layouts():
    from gen_worker_amd import _native
    from gen_worker_amd.flux_dit import attention

    q, k, v = _inputs(64, 96, 2, seed=1)
    with pytest.raises(ValueError, match="keys"):
        attention(q, k, v[:90])                         # 96 keys, 90 values
    with pytest.raises(ValueError, match="unit head"):
        attention(q.transpose(0, 1).contiguous().transpose(0, 1), k, v)
    lib = _native.load()
    rc = lib.gwa_dit_attention(None, 128, None, 128, None, 128, None, 128, 4, 4, 1, 64, 0.1, None)
    assert rc == 1 and "head_dim" in lib.gwa_last_error().decode()
