"""CPU tests of the nvfp4 compatibility lane: the oracle pinned against brute force, a library cast and the
reference's layout definition; the host-side format functions against the oracle; the op refusals."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nvfp4_oracle as N


def _all_e4m3_values():
    codes = np.arange(0, 0x7F, dtype=np.int64)   # 0x7F is NaN in e4m3fn
    return codes, N.e4m3_value(codes)


def test_e4m3_rne_is_the_nearest_code_ties_to_even():
    """Brute force over all finite non-negative codes, on midpoints, quarter points and random values."""
    codes, vals = _all_e4m3_values()
    rng = np.random.default_rng(0)
    mids = ((vals[1:].astype(np.float64) + vals[:-1]) / 2).astype(np.float32)
    quarters = ((vals[1:].astype(np.float64) * 3 + vals[:-1]) / 4).astype(np.float32)
    rand = np.exp(rng.uniform(np.log(2.0 ** -9), np.log(448.0), 20000)).astype(np.float32)
    x = np.concatenate([vals[1:], mids, quarters, rand])
    x = x[(x >= 2.0 ** -9) & (x <= 448.0)]
    d = np.abs(vals[None, :].astype(np.float64) - x[:, None].astype(np.float64))
    best = d.min(axis=1, keepdims=True)
    cand = (d == best)
    # nearest; between two equally near codes the even one
    want = np.array([c[np.flatnonzero(row)][0] if row.sum() == 1 else
                     [cc for cc in c[np.flatnonzero(row)] if cc % 2 == 0][0] for row, c in
                     zip(cand, np.broadcast_to(codes, cand.shape))], np.int64)
    assert np.array_equal(N.e4m3_rne(x).astype(np.int64), want)


def test_e4m3_rne_matches_torch_cast():
    """The library's float8_e4m3fn conversion (round to nearest even) agrees on the clamped range."""
    rng = np.random.default_rng(1)
    x = np.exp(rng.uniform(np.log(2.0 ** -9), np.log(448.0), 200000)).astype(np.float32)
    t = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(N.e4m3_rne(x), t)
    assert np.array_equal(N.e4m3_value(t), torch.from_numpy(t).view(torch.float8_e4m3fn).float().numpy())


def test_cast_e2m1_nearest_and_documented_ties():
    """Away from the bounds a code is the nearest e2m1 magnitude; on the seven bounds the reference's
    documented choices (0.75, 1.75 and 2.5 round up, the other four down); the sign is bit 3 (not for -0)."""
    rng = np.random.default_rng(2)
    q = rng.uniform(-7, 7, 50000).astype(np.float32)
    q = q[np.all(np.abs(np.abs(q)[:, None] - N.BOUNDS[None, :]) > 1e-3, axis=1)]
    c = N.cast_e2m1(q)
    mag = N.E2M1[c & 7]
    nearest = N.E2M1[np.argmin(np.abs(np.abs(q)[:, None] - N.E2M1[None, :]), axis=1)]
    assert np.array_equal(mag, nearest)
    assert np.array_equal(c >> 3, (q < 0).astype(np.uint8))
    b = N.BOUNDS
    assert N.cast_e2m1(b).tolist() == [0, 2, 2, 4, 5, 5, 6]
    assert N.cast_e2m1(-b).tolist() == [8, 10, 10, 12, 13, 13, 14]
    assert N.cast_e2m1(np.array([0.0, -0.0, 6.0, 9.0, -100.0], np.float32)).tolist() == [0, 0, 7, 7, 15]


def test_blocked_layout_matches_the_reference_definition():
    """The index loop equals the reference's definition as reshapes: pad to 128 x 4, tiles (row block, column
    block), each tile's rows split 4 x 32 and the two row factors swapped (to_blocked_scales,
    models/nvfp4_quant.py:72-84)."""
    rng = np.random.default_rng(3)
    for rows, kb in [(1, 1), (128, 4), (130, 7), (333, 192), (256, 3)]:
        flat = rng.integers(1, 255, (rows, kb), dtype=np.uint8)
        nrb, ncb = (rows + 127) // 128, (kb + 3) // 4
        pad = np.zeros((nrb * 128, ncb * 4), np.uint8)
        pad[:rows, :kb] = flat
        want = pad.reshape(nrb, 128, ncb, 4).transpose(0, 2, 1, 3).reshape(-1, 4, 32, 4).transpose(0, 2, 1, 3)
        got = N.to_blocked_scales(flat)
        assert np.array_equal(got, want.reshape(-1)), (rows, kb)
        assert np.array_equal(N.from_blocked_scales(got, rows, kb), flat)


def _blocks(rng, m, k, scale=1.0):
    return (rng.standard_normal((m, k)) * scale).astype(np.float32)


@pytest.mark.parametrize("m,k,s2", [(16, 64, 2.0 ** -10), (77, 512, 0.003), (5, 3072, 1.7e-4)])
def test_activation_quantizer_invariants(m, k, s2):
    """Per block: the largest magnitude maps to code 7 (6.0) unless the scale clamps; a zero block takes the
    smallest scale and zero codes; every code is within half an e2m1 step of x / (scale * s2); the element
    order of the packing; dequantized values quantize back to the same codes and scales."""
    rng = np.random.default_rng(m + k)
    x = N.bf16_round(_blocks(rng, m, k))
    x[0, :16] = 0.0                                   # a zero block: scale clamps to 2^-9, codes 0
    q, sc = N.quantize_activation(x, s2)
    assert q.shape == (m, k // 2) and sc.shape == (m, k // 16)
    codes = np.empty((m, k), np.uint8)
    codes[:, 0::2], codes[:, 1::2] = q & 0xF, q >> 4
    sa = N.e4m3_value(sc)
    den = (sa * np.float32(s2)).astype(np.float32)
    xb = x.reshape(m, k // 16, 16)
    cb = codes.reshape(m, k // 16, 16)
    t = np.abs(xb).max(-1) / np.float32(6.0 * np.float32(s2))
    free = (t > 2.0 ** -9) & (t < 448.0)
    top = np.take_along_axis(cb, np.abs(xb).argmax(-1)[..., None], -1)[..., 0] & 7
    assert np.all(top[free] == 7)
    assert np.all(codes.reshape(m, k // 16, 16)[0, 0] == 0) and sc[0, 0] == 1   # 2^-9 is code 1
    val = np.where(cb & 8, -1.0, 1.0) * N.E2M1[cb & 7]
    step = np.array([0.5, 0.5, 0.5, 0.5, 1.0, 1.0, 2.0, 2.0], np.float32)[cb & 7]
    r = xb / den[..., None]
    assert np.all((np.abs(val - np.clip(r, -6, 6)) <= step / 2 + 1e-6))
    # dequantized values quantize back to the same codes and scales (idempotence on the grid; a negative
    # value that rounds to zero keeps its sign bit, code 8, and comes back as +0, code 0)
    xdq = N.bf16_round(N.dequantize(q, sc, s2))
    q2, sc2 = N.quantize_activation(xdq, s2)

    def unsigned_zero(p):
        lo, hi = p & 0xF, p >> 4
        lo = np.where(lo == 8, 0, lo)
        hi = np.where(hi == 8, 0, hi)
        return (hi << 4) | lo

    keep = free[:, :, None].repeat(8, axis=2).reshape(m, k // 2)
    assert np.array_equal(unsigned_zero(q2)[keep], unsigned_zero(q)[keep])
    assert np.array_equal(sc2[free], sc[free])


def test_product_weight_quantizer_and_layouts_match_the_oracle():
    """gen_worker_amd.nvfp4.quantize_nvfp4_tensor (torch) == the oracle, zero blocks and rows included; the
    torch blocked-layout functions == the oracle's loop."""
    from gen_worker_amd import nvfp4

    rng = np.random.default_rng(4)
    w = (rng.standard_normal((96, 320)) * 0.05).astype(np.float32)
    w[3] = 0.0
    w[7, 16:32] = 0.0
    q, s, ws2 = nvfp4.quantize_nvfp4_tensor(torch.from_numpy(w))
    oq, os_, ows2 = N.quantize_nvfp4_tensor(w)
    assert np.array_equal(q.numpy(), oq)
    assert np.array_equal(s.view(torch.uint8).numpy(), os_)
    assert np.float32(ws2.item()) == ows2
    b = nvfp4.to_blocked_scales(s)
    assert np.array_equal(b.view(torch.uint8).numpy(), N.to_blocked_scales(os_))
    assert torch.equal(nvfp4.from_blocked_scales(b, 96, 20).view(torch.uint8), s.view(torch.uint8))


def test_nvfp4_ops_refuse_cpu_and_bad_shapes():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import nvfp4
    from gen_worker_amd.ops import SvdqOpError

    with pytest.raises(SvdqOpError, match="GPU only"):
        torch.ops.cozy_gen_worker.nvfp4_quant_act(torch.zeros(4, 32, dtype=torch.bfloat16), torch.ones(()), False,
                                                   False)
    with pytest.raises(SvdqOpError, match="GPU only"):   # a valid contract still needs the HIP kernels
        nvfp4.build_nvfp4_linear(torch.zeros(16, 8, dtype=torch.uint8), torch.zeros(16, 1, dtype=torch.uint8),
                                 torch.ones(()), device="cpu")
    with pytest.raises(nvfp4.Nvfp4Error, match="entries"):
        nvfp4.build_nvfp4_linear(torch.zeros(16, 16, dtype=torch.uint8), torch.zeros(16, 3, dtype=torch.uint8),
                                 torch.ones(()), device="cpu")


def test_nvfp4_fake_impls():
    import gen_worker_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(77, 384, dtype=torch.bfloat16)
        q, s, d = torch.ops.cozy_gen_worker.nvfp4_quant_act(x, torch.empty(()), True, True)
        assert q.shape == (77, 192) and s.shape == (128 * 24,) and d.shape == (77, 384)
        q3, s3, d3, sd = torch.ops.cozy_gen_worker.nvfp4_quant_act_dyn(x, False, False)
        assert s3.shape == (77, 24) and d3.shape == (0, 384) and sd.shape == ()
        q2, s2 = torch.ops.cozy_gen_worker.quant_nvfp4_act(x, torch.empty(()))
        assert s2.dtype == torch.float8_e4m3fn and s2.shape == (128 * 24,)
        w = torch.ops.cozy_gen_worker.nvfp4_dequant(torch.empty(64, 96, dtype=torch.uint8),
                                                    torch.empty(64, 12, dtype=torch.uint8), False)
        assert w.shape == (64, 192) and w.dtype == torch.bfloat16


def test_nan_handling_matches_torch_ops():
    """Non-finite inputs follow the reference's torch ops: amax and clamp keep a NaN, the e4m3 cast of a NaN
    is 0x7F, searchsorted puts a NaN past every e2m1 bound (code 7, sign clear), an infinite block maximum
    clamps to 448 and its infinity takes code 7 with its sign."""
    assert int(torch.tensor([float("nan")]).to(torch.float8_e4m3fn).view(torch.uint8)[0]) == N.E4M3_NAN
    assert int(N.e4m3_rne(np.array([np.nan], np.float32))[0]) == N.E4M3_NAN
    assert np.isnan(N.e4m3_value(N.E4M3_NAN)) and not np.isnan(N.e4m3_value(0x7E))
    bounds = torch.tensor(N.BOUNDS)
    for v in (float("nan"), -float("nan"), float("inf"), -float("inf")):
        t = torch.tensor([v], dtype=torch.float32)
        want = int(torch.searchsorted(bounds, t.abs())[0]) + 8 * int(t[0] < 0)
        assert int(N.cast_e2m1(np.array([v], np.float32))[0]) == want
    x = np.ones((2, 32), np.float32)
    x[0, 3] = np.nan                       # block (0, 0) holds a NaN
    x[1, 20] = np.inf                      # block (1, 1) holds an infinity
    q, sc = N.quantize_activation(x, 1.0)
    vals = N.unpack_e2m1(q)                # e2m1 values of the codes
    assert sc[0, 0] == N.E4M3_NAN and (vals[0, :16] == 6.0).all()          # every quotient NaN -> code 7
    assert (vals[1, 16:] == np.where(x[1, 16:] == np.inf, 6.0, vals[1, 16:])).all() and vals[1, 20] == 6.0
    xt = torch.from_numpy(x)
    bmax = xt.reshape(2, 2, 16).abs().amax(-1)
    sa = (bmax / 6.0).clamp(min=2.0 ** -9, max=448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(sc, sa)
    assert np.isnan(N.dynamic_s2(x)) and N.dynamic_s2(np.ones((1, 16), np.float32)) == np.float32(1.0 / 2688.0)
    assert N.dynamic_s2(np.zeros((1, 16), np.float32)) == np.float32(1e-12)
