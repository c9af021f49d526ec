"""nunchaku svdq fp4 packaging, CPU side: the oracle's micro-scale packer pinned by the reference's own known
answer (``tests/test_svdq_official_layout_pgw770.py:145-149``), the product's decoders against the oracle's
packers, the dense fold recovering the exported weight (the reference's bound, ``:231-235``), the fused
split, the oracle's module forward pinned against the float64 composition of independently pinned pieces,
and the loader's routing of an fp4 artifact."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import nunchaku_layout_oracle as N
from oracle import nvfp4_oracle as F4
from test_svdq_artifact import _qc, _write

from gen_worker_amd import svdq_artifact as A
from gen_worker_amd import svdq_checkpoint as C
from gen_worker_amd import svdq_fp4 as S
from gen_worker_amd import synthetic


# ------------------------------------------------------------------ oracle pinning

def test_oracle_micro_scale_known_answer():
    """Every fourth stored byte of the first 128-row block holds row 32 (j % 4) + 8 ((j / 4) % 4) + j / 16:
    the (4, 4, 8) row split with the 8-row lane outermost."""
    n, nb = 256, 32
    idx = np.repeat(np.arange(n, dtype=np.int64)[:, None], nb, axis=1)
    order = N.pack_micro_scale(idx).reshape(-1)[:512:4]
    assert order.tolist() == [(j % 4) * 32 + ((j // 4) % 4) * 8 + (j // 16) for j in range(128)]
    # the four blocks of one row sit side by side; the next block quad follows the whole 128-row block
    blk = np.repeat(np.arange(nb, dtype=np.int64)[None, :], n, axis=0)
    stored = N.pack_micro_scale(blk).reshape(-1)
    assert stored[:8].tolist() == [0, 1, 2, 3, 0, 1, 2, 3] and stored[512:516].tolist() == [4, 5, 6, 7]
    assert stored[nb * 128] == 0                                    # row block 1 starts after all of block 0


def _e4m3_grid(n, nb, seed):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.uniform(1.0, 400.0, (n, nb)).astype(np.float32)).to(torch.float8_e4m3fn)


@pytest.mark.parametrize("n,k", [(128, 64), (256, 512), (384, 768)])
def test_micro_scale_pack_matches_the_oracle(n, k):
    flat = _e4m3_grid(n, k // 16, n + k)
    want = N.pack_micro_scale(flat.view(torch.uint8).numpy())
    assert np.array_equal(S.pack_micro_scales(flat).view(torch.uint8).numpy(), want)
    back = S.unpack_micro_scales(torch.from_numpy(want).view(torch.float8_e4m3fn), n, k)
    assert torch.equal(back.view(torch.uint8), flat.view(torch.uint8))


@pytest.mark.parametrize("n,k", [(9216, 3072), (3072, 3072), (12288, 3072), (3072, 12288)])
def test_micro_scale_roundtrip_at_the_model_shapes(n, k):
    flat = _e4m3_grid(n, k // 16, 7)
    stored = S.pack_micro_scales(flat)
    assert tuple(stored.shape) == (k // 16, n)
    assert torch.equal(S.unpack_micro_scales(stored, n, k).view(torch.uint8), flat.view(torch.uint8))
    # the (4, 8, 4) split reshapes without error and permutes rows: it must not decode the same
    wrong = stored.view(torch.uint8).reshape(n // 128, k // 64, 4, 8, 4, 4).permute(0, 4, 3, 2, 1, 5)
    assert not torch.equal(wrong.reshape(n, k // 16), flat.view(torch.uint8))


def test_micro_scale_refusals():
    with pytest.raises(C.SvdqLayoutError, match="micro-scale"):
        S.unpack_micro_scales(torch.zeros(4, 96, dtype=torch.float8_e4m3fn), 96, 64)      # out % 128
    with pytest.raises(C.SvdqLayoutError, match="micro-scale"):
        S.unpack_micro_scales(torch.zeros(2, 128, dtype=torch.float8_e4m3fn), 128, 32)    # (in / 16) % 4
    with pytest.raises(C.SvdqLayoutError, match="shape"):
        S.unpack_micro_scales(torch.zeros(128, 4, dtype=torch.float8_e4m3fn), 128, 64)


# ------------------------------------------------------------------ decoding a linear

def _oracle_fp4_layer(n, k, rank, seed, *, per_channel):
    """Logical fp4 svdq tensors and their stored form, encoded by the oracle's packers."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    scales = torch.from_numpy(rng.uniform(2e-3, 0.5, (n, k // 16)).astype(np.float32)).to(torch.float8_e4m3fn)
    bf = lambda a: torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)  # noqa: E731
    logical = dict(codes=codes, scales=scales, smooth=bf(rng.uniform(0.5, 2.0, k)), bias=bf(rng.normal(0, .02, n)),
                   down=bf(rng.normal(0, 0.02, (k, rank))), up=bf(rng.normal(0, 0.02, (n, rank))))
    stored = {
        "qweight": torch.from_numpy(N.pack_weight(codes)),
        "wscales": torch.from_numpy(N.pack_micro_scale(scales.view(torch.uint8).numpy())).view(torch.float8_e4m3fn),
        "smooth_factor": bf(N.pack_scale(logical["smooth"].float().numpy().reshape(-1, 1)).reshape(-1)),
        "bias": bf(N.pack_scale(logical["bias"].float().numpy().reshape(-1, 1)).reshape(-1)),
        "proj_down": bf(N.pack_lowrank(logical["down"].float().numpy(), down=True)),
        "proj_up": bf(N.pack_lowrank(logical["up"].float().numpy(), down=False)),
    }
    if per_channel:
        sc = bf(rng.uniform(1e-4, 1e-3, n))
        logical["second"] = sc.float()
        stored["wcscales"] = bf(N.pack_scale(sc.float().numpy().reshape(-1, 1)).reshape(-1))
    else:
        logical["second"] = torch.tensor([3e-4]).to(torch.bfloat16).float()
        stored["wtscale"] = logical["second"].to(torch.bfloat16)
    return logical, stored


@pytest.mark.parametrize("per_channel", [True, False], ids=["wcscales", "wtscale"])
def test_decode_fp4_linear_matches_logical(per_channel):
    logical, stored = _oracle_fp4_layer(256, 384, 32, 5, per_channel=per_channel)
    assert S.is_fp4_svdq_linear(stored) and not C.is_int4_svdq_linear(stored)
    dec = S.decode_fp4_linear(stored, 256, 384)
    assert dec.rank == 32 and (dec.out_features, dec.in_features) == (256, 384)
    assert np.array_equal(dec.codes.numpy(), logical["codes"])
    assert torch.equal(dec.scales.view(torch.uint8), logical["scales"].view(torch.uint8))
    assert torch.equal(dec.second.reshape(-1), logical["second"].reshape(-1))
    for key, got in (("smooth", dec.smooth_factor), ("bias", dec.bias), ("down", dec.proj_down),
                     ("up", dec.proj_up)):
        assert torch.equal(got, logical[key]), key
    # dequantization: e2m1(code) * micro-scale * second, from the oracle's decoders
    w = F4.dequantize(F4.pack_e2m1(logical["codes"]), logical["scales"].view(torch.uint8).numpy())
    w = w * logical["second"].numpy().reshape(-1, 1)
    assert np.array_equal(C.dequantize_decoded(dec).numpy(), w.astype(np.float32))


def test_decode_fp4_refusals():
    _, stored = _oracle_fp4_layer(128, 128, 16, 1, per_channel=True)
    with pytest.raises(C.SvdqLayoutError, match="neither wcscales nor wtscale"):
        S.decode_fp4_linear({k: v for k, v in stored.items() if k != "wcscales"}, 128, 128)
    with pytest.raises(C.SvdqLayoutError, match="wcscales numel"):
        S.decode_fp4_linear(dict(stored, wcscales=stored["wcscales"][:64]), 128, 128)
    with pytest.raises(C.SvdqLayoutError, match="one half"):
        S.decode_fp4_linear({k: v for k, v in stored.items() if k != "proj_up"}, 128, 128)
    with pytest.raises(C.SvdqLayoutError, match="not an fp4"):
        S.decode_fp4_linear(dict(stored, wscales=torch.zeros(2, 128, dtype=torch.float16)), 128, 128)
    with pytest.raises(C.SvdqLayoutError, match="missing"):
        S.decode_fp4_linear({"qweight": stored["qweight"]}, 128, 128)
    # an fp4 linear is not an int4 one, and the int4 decoder says so
    with pytest.raises(C.SvdqLayoutError, match="not an int4"):
        C.decode_int4_linear(stored, 128, 128)


def _rel(a, b):
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("n,k,per_channel,smooth", [(3072, 3072, False, False), (3072, 3072, False, True),
                                                    (9216, 3072, True, True), (1536, 6144, False, True)])
def test_dense_fold_recovers_the_exported_weight(n, k, per_channel, smooth):
    """The fold W / s + up @ (down / s)^T reconstructs the exporter's W within fp4 quantization error (the
    reference's own bound for this check is 0.35)."""
    L = synthetic.svdq_fp4_layer(n, k, 128, per_channel=per_channel, smooth=smooth, seed_offset=n + k)
    dec = S.decode_fp4_linear(L.stored, n, k)
    assert (dec.second.numel() > 1) == per_channel
    lin = C.fold_decoded(dec, compute_dtype=torch.float32)
    err = _rel(lin.weight.detach(), L.w)
    assert err < 0.35, err
    assert err < 0.15, f"fp4 g16 on a Gaussian residual should land near 0.1 of it, got {err}"
    assert torch.equal(lin.bias.detach(), L.bias.float())
    # a wrong fold (the low-rank branch dropped, or the smoothing not undone) misses by far more
    deq = C.dequantize_decoded(dec)
    assert _rel(deq / dec.smooth_factor.float().reshape(1, -1) if smooth else deq, L.w) > 4 * err
    if smooth:
        assert _rel(deq + dec.proj_up.float() @ dec.proj_down.float().t(), L.w) > 4 * err


def test_split_fp4_keeps_the_decoded_order():
    L = synthetic.svdq_fp4_layer(3 * 1024, 1024, 32, per_channel=True, seed_offset=11)
    dec = S.decode_fp4_linear(L.stored, 3 * 1024, 1024)
    parts = C.split_decoded(dec, (1024, 1024, 1024))
    full = C.dequantize_decoded(dec)
    for i, part in enumerate(parts):
        assert isinstance(part, S.DecodedFp4Linear) and part.proj_down is dec.proj_down
        assert torch.equal(C.dequantize_decoded(part), full[i * 1024:(i + 1) * 1024])
        assert torch.equal(part.bias, L.bias[i * 1024:(i + 1) * 1024])
        assert _rel(C.fold_decoded(part, compute_dtype=torch.float32).weight.detach(),
                    L.w[i * 1024:(i + 1) * 1024]) < 0.15


# ------------------------------------------------------------------ the oracle's module forward

def _oracle_inputs(L, n, k, m, seed):
    dec = S.decode_fp4_linear(L.stored, n, k)
    x = synthetic.activation(m, k, outlier_frac=0.01, outlier_scale=20.0, seed=seed).float().numpy()
    wq = F4.pack_e2m1(dec.codes.numpy())
    ws = dec.scales.view(torch.uint8).numpy()
    return dec, x, wq, ws


def _f(t):
    return None if t is None else t.float().numpy()


def test_oracle_svdq_fp4_forward_is_the_quantized_composition():
    """The oracle forward = (deq(Q(x / s)) * s2) @ (deq(W) * second)^T + (x @ down) @ up^T + bias up to the
    bf16 roundings between the steps; Q, deq and s2 are the nvfp4 pieces pinned by the nvfp4 tests. Each
    plausible slip (a scale, the smoothing, the branch or the bias dropped; the branch fed the smoothed
    input) misses by far more."""
    n, k, m = 256, 512, 64
    L = synthetic.svdq_fp4_layer(n, k, 32, per_channel=True, seed_offset=3)
    dec, x, wq, ws = _oracle_inputs(L, n, k, m, 41)
    sm, sec, down, up = _f(dec.smooth_factor), dec.second.numpy(), _f(dec.proj_down), _f(dec.proj_up)
    b = F4.bf16_round(_f(dec.bias) * 100.0)            # a bias on the outputs' own scale, so dropping it shows
    got = F4.svdq_fp4_linear(x, sm, wq, ws, sec, down, up, b)

    xs = F4.bf16_round(x / sm.reshape(1, -1))
    s2 = F4.dynamic_s2(xs)
    xq, xsc = F4.quantize_activation(xs, s2)
    xd = F4.dequantize(xq, xsc, s2).astype(np.float64)
    wd = F4.dequantize(wq, ws).astype(np.float64) * sec.reshape(-1, 1).astype(np.float64)
    want = xd @ wd.T + (x.astype(np.float64) @ down) @ up.T + b

    def rel(a):
        return float(np.linalg.norm(a - want) / np.linalg.norm(want))
    assert rel(got) < 4e-3, rel(got)
    slips = {
        "no second": F4.svdq_fp4_linear(x, sm, wq, ws, np.ones_like(sec) * sec.mean(), down, up, b),
        "no smoothing": F4.svdq_fp4_linear(x, None, wq, ws, sec, down, up, b),
        "no branch": F4.svdq_fp4_linear(x, sm, wq, ws, sec, None, None, b),
        "no bias": F4.svdq_fp4_linear(x, sm, wq, ws, sec, down, up, None),
        "branch on x / s": F4.svdq_fp4_linear(x, sm, wq, ws, sec, None, None, b)
        + F4.bf16_round(F4.bf16_round(xs @ down) @ up.T),
    }
    for name, y in slips.items():
        assert rel(y) > 10 * 4e-3, f"{name}: {rel(y)}"


def test_oracle_svdq_fp4_forward_recovers_the_exported_linear():
    """End to end: the oracle forward on an exported layer approximates x @ W^T + bias within W4A4 fp4
    error (weight and activation both at 4 bits)."""
    n, k, m = 512, 1024, 96
    L = synthetic.svdq_fp4_layer(n, k, 32, per_channel=False, seed_offset=5)
    dec, x, wq, ws = _oracle_inputs(L, n, k, m, 43)
    got = F4.svdq_fp4_linear(x, _f(dec.smooth_factor), wq, ws, dec.second.numpy(), _f(dec.proj_down),
                             _f(dec.proj_up), _f(dec.bias))
    want = x.astype(np.float64) @ L.w.double().numpy().T + L.bias.double().numpy()
    err = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    assert err < 0.25, err


# ------------------------------------------------------------------ modes, modules and the loader

def test_fp4_modes():
    assert S.resolve_fp4_mode(None) == "dense" and S.resolve_fp4_mode("") == "dense"
    assert S.resolve_fp4_mode("blockwise") == "blockwise"
    with pytest.raises(C.SvdqLayoutError, match="fp4 mode"):
        S.resolve_fp4_mode("fused")
    assert S.fp4_shape_supported(3072, 3072) and not S.fp4_shape_supported(3072, 3056)
    assert not S.fp4_shape_supported(3080, 3072)


def test_blockwise_module_runs_on_the_gpu_only():
    """No CPU fallback: building the blockwise module off the GPU fails in the HIP op's device check."""
    L = synthetic.svdq_fp4_layer(128, 128, 16, seed_offset=2)
    dec = S.decode_fp4_linear(L.stored, 128, 128)
    with pytest.raises(Exception, match="cuda|GPU|device"):
        S.build_fp4_module(dec, device="cpu", mode="blockwise")
    assert isinstance(S.build_fp4_module(dec, device="cpu"), nn.Linear)


class _Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.to_q, self.to_k, self.to_v = nn.Linear(d, d), nn.Linear(d, d), nn.Linear(d, d)
        self.to_out = nn.ModuleList([nn.Linear(d, d)])


def _fp4_snapshot(tmp_path, d, rank):
    qkv = synthetic.svdq_fp4_layer(3 * d, d, rank, per_channel=True, seed_offset=21)
    out = synthetic.svdq_fp4_layer(d, d, rank, per_channel=False, seed_offset=22)
    tensors = {f"blocks.0.attn.to_qkv.{k}": v.contiguous() for k, v in qkv.stored.items()}
    tensors.update({f"blocks.0.attn.to_out.0.{k}": v.contiguous() for k, v in out.stored.items()})
    tensors["blocks.0.scale_table"] = torch.arange(4.0)
    meta = {"model_class": "NunchakuFluxTransformer2DModel", "quantization_config": _qc("fp4_e2m1_all", rank)}
    _write(tmp_path / "snap" / "transformer" / "svdq.safetensors", meta, tensors)
    return qkv, out


def _skeleton(d):
    class _Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = _Attn(d)
            self.register_buffer("scale_table", torch.zeros(4))

    model = nn.Module()
    model.blocks = nn.ModuleList([_Block()])
    return model


def test_load_fp4_artifact_dense_mode(tmp_path):
    d = 256
    qkv, out = _fp4_snapshot(tmp_path, d, 32)
    model = _skeleton(d)
    counts = A.load_svdq_artifact(tmp_path / "snap", model, device="cpu", lane="dense")
    assert counts["artifact"].precision == "fp4" and counts["fp4_mode"] == "dense"
    assert counts["fp4_prefixes"] == 2 and counts["int4_prefixes"] == 0
    assert counts["linears"] == 4 and counts["dense"] == 4 and counts["plain"] == 1
    attn = model.blocks[0].attn
    parts = C.split_decoded(S.decode_fp4_linear(qkv.stored, 3 * d, d), (d, d, d))
    for mod, part in zip((attn.to_q, attn.to_k, attn.to_v), parts):
        assert torch.equal(mod.weight, C.fold_decoded(part, device="cpu").weight)
    assert torch.equal(attn.to_out[0].weight, C.fold_decoded(S.decode_fp4_linear(out.stored, d, d)).weight)
    assert torch.equal(model.blocks[0].scale_table, torch.arange(4.0))


def test_fp4_artifact_refusals(tmp_path):
    d = 128
    _fp4_snapshot(tmp_path, d, 16)
    with pytest.raises(C.SvdqLayoutError, match="fp4 mode"):
        A.load_svdq_artifact(tmp_path / "snap", _skeleton(d), device="cpu", lane="dense", fp4_mode="fused")
    # a linear stored in the other precision than the artifact declares
    f = tmp_path / "snap" / "transformer" / "svdq.safetensors"
    with pytest.raises(C.SvdqLayoutError, match="declares svdq-int4"):
        C.load_svdq_checkpoint(f, _skeleton(d), device="cpu", lane="dense", precision="int4")
