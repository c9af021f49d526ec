"""The DiT block glue kernels (csrc/dit_block.hip) against the torch expressions the model states them with
(``gen_worker_amd.flux_dit``: ``_rms``, ``_rope``, ``_ln``): the gated residual bit for bit (elementwise, the
same two roundings); the qk norm + rotary and the adaLN modulation bit for bit except where the fp32 sum
of a row (mean of squares, mean and variance), added in another order than torch's reduction kernels, lands
the next bf16 rounding on the other side of a tie: such elements are rare (< 1e-3) and one or two bf16
steps away, counted at the magnitude of the last rounding's operands (the last add or subtract can cancel).
Shapes: the full-size DiT's (4096 image + 512 text tokens, hidden 3072, 24 heads) and ragged
small ones, with the row strides the model uses (column slices of a fused qkv output, row slices of the
joint sequence)."""

from __future__ import annotations

import pytest
import torch

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native

    _native.load()
    yield


def _bf16_steps(a: torch.Tensor, b: torch.Tensor, mag: torch.Tensor) -> torch.Tensor:
    """|a - b| in units of the bf16 spacing at mag (bf16 has 8 significant bits)."""
    a, b = a.double(), b.double()
    mag = torch.maximum(mag.double().abs(), torch.maximum(a.abs(), b.abs())).clamp_min(2.0 ** -126)
    return (a - b).abs() / torch.exp2(torch.floor(torch.log2(mag)) - 7)


def _close(got: torch.Tensor, want: torch.Tensor, what: str, mag: torch.Tensor, max_frac: float = 1e-3,
           max_steps: float = 4.0):
    """At most max_frac of the elements differ, each by at most max_steps bf16 steps at mag (the magnitude
    of the operands of the expression's last rounding)."""
    assert got.shape == want.shape and got.dtype == want.dtype == torch.bfloat16
    diff = got != want
    frac = diff.float().mean().item()
    steps = _bf16_steps(got[diff], want[diff], mag[diff]).max().item() if diff.any() else 0.0
    print(f"{what}: {int(diff.sum())} of {got.numel()} differ, at most {steps:.2f} bf16 steps")
    assert frac <= max_frac and steps <= max_steps, (what, frac, steps)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,pad", [(4096, 3072, 0), (77, 512, 64), (5, 3072, 8)])
def test_gate_residual_bit_exact(rows, cols, pad):
    from gen_worker_amd.flux_dit import gate_residual

    g = torch.Generator(device=DEV).manual_seed(rows + cols)
    xb = torch.randn(rows, cols + pad, generator=g, device=DEV).to(torch.bfloat16)
    x = xb[:, :cols]                                          # row stride cols + pad
    y = (torch.randn(rows, cols, generator=g, device=DEV) * 3).to(torch.bfloat16)
    gate = torch.randn(1, 6 * cols, generator=g, device=DEV).to(torch.bfloat16).chunk(6, dim=-1)[2]
    got = gate_residual(x, y, gate)
    want = x + gate * y
    assert torch.equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", [(4096, 3072), (512, 3072), (77, 512), (3, 1024)])
def test_adaln_modulate(rows, cols):
    from gen_worker_amd.flux_dit import _ln, adaln_modulate

    g = torch.Generator(device=DEV).manual_seed(7 * rows + cols)
    x = (torch.randn(rows, cols, generator=g, device=DEV) * 4 + 1).to(torch.bfloat16)
    x[:, 5] *= 30                                             # an outlier channel
    mod = (torch.randn(1, 6 * cols, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    sh, sc = mod.chunk(6, dim=-1)[:2]
    got = adaln_modulate(x, sc, sh)
    prod = _ln(x) * (1 + sc)
    want = prod + sh
    _close(got, want, f"adaln {rows}x{cols}", torch.maximum(prod.abs(), sh.abs().expand_as(prod)))
    # a row slice of a larger activation (the final norm reads the image rows of the joint sequence)
    got2 = adaln_modulate(x[1:], sc, sh)
    assert torch.equal(got2, got[1:])


@pytest.mark.gpu
@pytest.mark.parametrize("rows,heads,pos0,off", [(4096, 24, 512, 0), (512, 24, 0, 0), (67, 4, 3, 0),
                                                (33, 6, 1, 0), (29, 6, 2, 2)])
def test_qk_norm_rope(rows, heads, pos0, off):
    """Aligned rows take the wide kernel (4 heads per wave; 6 heads: a half-empty second group); off = 2
    (rows 4-byte aligned only) the one-head-per-wave kernel."""
    from gen_worker_amd.flux_dit import _rms, _rope, qk_norm_rope

    d, c = 128, heads * 128
    g = torch.Generator(device=DEV).manual_seed(rows * heads + pos0)
    qkv = (torch.randn(rows, 3 * c + off, generator=g, device=DEV) * 2).to(torch.bfloat16)[:, off:]
    qkv[:, 7] *= 40
    wq = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(torch.bfloat16)
    npos = pos0 + rows + 5
    inv = 1.0 / (10000.0 ** (torch.arange(d // 2, device=DEV, dtype=torch.float32) / (d // 2)))
    ang = torch.arange(npos, device=DEV, dtype=torch.float32)[:, None] * inv[None, :]
    cos = ang.cos().to(torch.bfloat16).unsqueeze(1)
    sin = ang.sin().to(torch.bfloat16).unsqueeze(1)
    # outputs are rows [2, 2 + rows) of a joint buffer
    q, k, v = (torch.full((rows + 4, heads, d), 7.0, device=DEV, dtype=torch.bfloat16) for _ in range(3))
    sl = slice(2, 2 + rows)
    qk_norm_rope(qkv[:, :c], qkv[:, c:2 * c], wq, wk, cos, sin, pos0, q[sl], k[sl], v=qkv[:, 2 * c:], out_v=v[sl])
    hq = (rows, heads, d)
    cs, sn = cos[pos0:pos0 + rows], sin[pos0:pos0 + rows]
    for name, got, src, w in (("q", q[sl], qkv[:, :c], wq), ("k", k[sl], qkv[:, c:2 * c], wk)):
        y = _rms(src.reshape(hq), w)
        pair = torch.maximum(y[..., 0::2].abs(), y[..., 1::2].abs())      # rotary terms are at most this
        _close(got, _rope(y, cs, sn), f"{name} {rows}x{heads}", pair.repeat_interleave(2, dim=-1))
    assert torch.equal(v[sl], qkv[:, 2 * c:].reshape(hq))
    for t in (q, k, v):                                       # rows outside the slice untouched
        assert bool((t[:2] == 7).all()) and bool((t[2 + rows:] == 7).all())


@pytest.mark.gpu
def test_glue_wrappers_refuse_bad_layouts():
    from gen_worker_amd.flux_dit import adaln_modulate, gate_residual, qk_norm_rope

    x = torch.zeros(8, 512, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="unit column stride"):
        adaln_modulate(x.t(), x[0, :8], x[0, :8])
    with pytest.raises(ValueError, match="contiguous bf16"):
        adaln_modulate(x, x[0, :256], x[0])
    with pytest.raises(ValueError, match="rows"):
        gate_residual(x, x[:4], x[0])
    q = torch.zeros(8, 2, 128, device=DEV, dtype=torch.bfloat16)
    tab = torch.zeros(8, 1, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.ones(128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="v and out_v"):
        qk_norm_rope(x[:, :256], x[:, 256:], w, w, tab, tab, 0, q, q.clone(), v=x[:, :256])
