"""GPU parity of the nvfp4 compatibility lane: activation codes, e4m3 scales (flat and blocked) and the
dequantized activations bit for bit against the oracle, the reference's identity-probe shapes included; the
weight decode bit for bit; the module forward against the oracle's forward within the output tolerance."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import check_output
from oracle import nvfp4_oracle as N

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import gen_worker_amd  # noqa: F401  (registers the ops)
    from gen_worker_amd import _native

    _native.load()
    yield


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(N.bf16_round(a)).to(torch.bfloat16).to(DEV)


def _act(m, k, seed, outliers=True):
    g = np.random.default_rng(seed)
    x = g.standard_normal((m, k)).astype(np.float32)
    if outliers:
        x[:, g.permutation(k)[: max(1, k // 100)]] *= 30.0
    return N.bf16_round(x)


def _edge_rows(k):
    """Rows whose quotients land exactly on every e2m1 bound (scale 1, s2 = 2^-10, so q = x * 2^10), a zero
    block, a negative-zero block, a huge block (scale clamps at 448) and a tiny one (clamps at 2^-9)."""
    s2 = 2.0 ** -10
    rows = []
    for sign in (1.0, -1.0):
        r = np.zeros(k, np.float32)
        blk = np.array([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 0.1, 5.5],
                       np.float32) * s2
        r[:16] = sign * blk
        r[16:32] = 0.0
        r[32:48] = -0.0
        if k >= 64:
            r[48:64] = sign * np.linspace(1e4, 3e4, 16, dtype=np.float32)
        rows.append(r)
    r = np.full(k, 1e-12, np.float32)
    rows.append(r)
    return N.bf16_round(np.stack(rows)), s2


@pytest.mark.parametrize("m,k", [(1, 16), (128, 512), (333, 3072), (1024, 12288), (77, 384), (130, 4112)])
@pytest.mark.parametrize("static", [True, False])
def test_quant_act_bit_exact(m, k, static):
    x = _act(m, k, seed=m + k)
    xd = _bf16(x)
    if static:
        s2v = np.float32(0.0037)
        s2 = torch.tensor(s2v, dtype=torch.float32, device=DEV)
    else:   # the reference's formula (models/w4a4.py:342-343) in float32 on the CPU
        s2v = np.float32(max(np.float32(np.abs(x).max()) / np.float32(2688.0), np.float32(1e-12)))
        s2 = None
    print(f"nvfp4 act-quant: M={m} K={k} s2={s2v} static={static}", flush=True)
    if static:
        q, sc, xdq = torch.ops.cozy_gen_worker.nvfp4_quant_act(xd, s2, False, True)
        qb, scb, _ = torch.ops.cozy_gen_worker.nvfp4_quant_act(xd, s2, True, False)
    else:
        q, sc, xdq, s2d = torch.ops.cozy_gen_worker.nvfp4_quant_act_dyn(xd, False, True)
        qb, scb, _, _ = torch.ops.cozy_gen_worker.nvfp4_quant_act_dyn(xd, True, False)
        assert np.float32(s2d.item()) == s2v
    oq, osc = N.quantize_activation(x, s2v)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(sc.cpu().numpy(), osc)
    assert torch.equal(qb, q)
    assert np.array_equal(scb.cpu().numpy(), N.to_blocked_scales(osc))
    want = N.dequantize(oq, osc)
    assert np.array_equal(xdq.float().cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_quant_act_edge_values():
    x, s2v = _edge_rows(128)
    s2 = torch.tensor(s2v, dtype=torch.float32, device=DEV)
    q, sc, xdq = torch.ops.cozy_gen_worker.nvfp4_quant_act(_bf16(x), s2, False, True)
    oq, osc = N.quantize_activation(x, s2v)
    assert np.array_equal(q.cpu().numpy(), oq) and np.array_equal(sc.cpu().numpy(), osc)
    # the first block: the quotients sit exactly on the bounds; the reference's tie choices
    codes = np.stack([oq[0, :8] & 0xF, oq[0, :8] >> 4], 1).reshape(-1)
    assert codes[:8].tolist() == [7, 0, 2, 2, 4, 5, 5, 6]
    assert osc[0, 0] == 0x38 and osc[0, 3] == 0x7E and osc[2, 0] == 1   # 1.0, 448, 2^-9
    assert np.array_equal(xdq.float().cpu().numpy().view(np.uint32), N.dequantize(oq, osc).view(np.uint32))


def test_quant_act_non_finite():
    """NaN and infinite inputs take the reference's values: a block holding a NaN gets the e4m3 NaN scale
    (0x7F) and code 7 everywhere, an infinity clamps its block scale to 448 and takes code 7 with its sign;
    with the dynamic second-level scale one NaN makes s2 NaN and every block NaN."""
    x = _act(4, 64, seed=3)
    x[0, 5] = np.nan
    x[1, 17] = np.inf
    x[2, 40] = -np.inf
    s2v = np.float32(0.01)
    q, sc, xdq = torch.ops.cozy_gen_worker.nvfp4_quant_act(_bf16(x), torch.tensor(s2v, device=DEV), False, True)
    oq, osc = N.quantize_activation(x, s2v)
    assert np.array_equal(q.cpu().numpy(), oq) and np.array_equal(sc.cpu().numpy(), osc)
    assert osc[0, 0] == N.E4M3_NAN and osc[1, 1] == 0x7E and osc[2, 2] == 0x7E
    got, want = xdq.float().cpu().numpy(), N.dequantize(oq, osc)
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.isnan(got[0, :16]).all()
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    q2, sc2, xdq2, s2d = torch.ops.cozy_gen_worker.nvfp4_quant_act_dyn(_bf16(x), False, True)
    assert np.isnan(s2d.item()) and np.isnan(N.dynamic_s2(x))
    oq2, osc2 = N.quantize_activation(x, N.dynamic_s2(x))
    assert np.array_equal(q2.cpu().numpy(), oq2) and np.array_equal(sc2.cpu().numpy(), osc2)
    assert (osc2 == N.E4M3_NAN).all() and torch.isnan(xdq2.float()).all()


def test_reference_op_contract():
    """quant_nvfp4_act returns (codes, blocked e4m3 scales), the reference op's outputs."""
    x = _act(333, 3072, seed=5)
    s2 = torch.tensor(0.002, dtype=torch.float32, device=DEV)
    q, sb = torch.ops.cozy_gen_worker.quant_nvfp4_act(_bf16(x), s2)
    assert sb.dtype == torch.float8_e4m3fn and sb.numel() == N.blocked_scale_numel(333, 192)
    oq, osc = N.quantize_activation(x, np.float32(0.002))
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(sb.view(torch.uint8).cpu().numpy(), N.to_blocked_scales(osc))


@pytest.mark.parametrize("blocked", [False, True])
def test_weight_decode_bit_exact(blocked):
    g = np.random.default_rng(7)
    w = (g.standard_normal((300, 1024)) * 0.02).astype(np.float32)
    w[5] = 0.0
    oq, osc, _ = N.quantize_nvfp4_tensor(w)
    sc = N.to_blocked_scales(osc) if blocked else osc
    out = torch.ops.cozy_gen_worker.nvfp4_dequant(torch.from_numpy(oq).to(DEV), torch.from_numpy(sc).to(DEV),
                                                  blocked)
    assert np.array_equal(out.float().cpu().numpy().view(np.uint32), N.dequantize(oq, osc).view(np.uint32))


@pytest.mark.parametrize("m,n,k,static,pqs,bias", [(77, 768, 3072, False, False, True),
                                                   (256, 3072, 3072, True, False, True),
                                                   (40, 512, 1024, False, True, False)])
def test_module_matches_oracle(m, n, k, static, pqs, bias):
    """Nvfp4Linear built from the reference module's buffers (blocked weight scales) against the oracle forward
    (the fp4 product summed in float64, rounded to bf16, times bf16(s2 * ws2), plus the bias)."""
    from gen_worker_amd import nvfp4

    g = np.random.default_rng(m + n)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    oq, osc, ws2 = N.quantize_nvfp4_tensor(w)
    b = N.bf16_round((g.standard_normal(n) * 0.05).astype(np.float32)) if bias else None
    p = N.bf16_round(g.uniform(0.5, 2.0, k).astype(np.float32)) if pqs else None
    x = _act(m, k, seed=m * 3 + k)
    isc = np.float32(0.004) if static else None
    mod = nvfp4.build_nvfp4_linear(
        torch.from_numpy(oq), torch.from_numpy(N.to_blocked_scales(osc)).view(torch.float8_e4m3fn),
        torch.tensor([[ws2]], dtype=torch.float32),
        bias=None if b is None else torch.from_numpy(b).to(torch.bfloat16),
        input_scale=None if isc is None else torch.tensor([[isc]], dtype=torch.float32),
        pre_quant_scale=None if p is None else torch.from_numpy(p).to(torch.bfloat16), device=DEV)
    with torch.no_grad():
        y = mod(_bf16(x).reshape(1, m, k))
    assert y.shape == (1, m, n) and y.dtype == torch.bfloat16
    xin = N.bf16_round(x * p) if p is not None else x
    s2 = isc if static else np.float32(max(np.float32(np.abs(xin).max()) / np.float32(2688.0), np.float32(1e-12)))
    ref = N.nvfp4_linear(xin, s2, oq, osc, ws2, b)
    check_output(y.reshape(m, n), ref, what=f"nvfp4 module {m}x{n}x{k}")


@pytest.mark.parametrize("bias", [True, False])
def test_scale_bias_bit_exact(bias):
    """The one-pass epilogue == the reference's two bf16-rounded steps: RN(RN(y * RN(s2 * ws2)) + bias)."""
    g = np.random.default_rng(9)
    y = N.bf16_round((g.standard_normal((37, 264)) * 3).astype(np.float32))
    b = N.bf16_round((g.standard_normal(264) * 0.5).astype(np.float32))
    s2, ws2 = np.float32(0.0123), np.float32(0.0071)
    yd = _bf16(y)
    torch.ops.cozy_gen_worker.nvfp4_scale_bias(yd, torch.tensor(s2, device=DEV), torch.tensor(ws2, device=DEV),
                                               _bf16(b) if bias else None)
    want = N.bf16_round(y * N.bf16_round(s2 * ws2))
    if bias:
        want = N.bf16_round(want + b)
    assert np.array_equal(yd.float().cpu().numpy().view(np.uint32), want.view(np.uint32))
