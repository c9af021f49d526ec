"""nunchaku svdq int4 checkpoint layout, CPU side: the oracle's forward packers pinned by known answers
(the reference's own vector-order answer, ``tests/test_svdq_official_layout_pgw770.py:149``, and
hand-derived word / pack positions of the mma fragment structure), the product's decoders against the
oracle's packers, decoding a whole linear, the fused-projection split and the swap planning."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import nunchaku_layout_oracle as N

from gen_worker_amd import svdq_checkpoint as C


# ------------------------------------------------------------------ oracle pinning

def test_oracle_vector_order_known_answer():
    """The reference's known answer for pack_scale on a vector: [0, 1, 8, 9, 2, 3, 10, 11, ...]."""
    stored = N.pack_scale(np.arange(128, dtype=np.float32).reshape(128, 1)).reshape(-1)
    assert stored[:8].tolist() == [0, 1, 8, 9, 2, 3, 10, 11]
    # rows 16 apart (the 8 lane groups of a 128-row block) are 16 apart in storage
    assert stored[16:24].tolist() == [16, 17, 24, 25, 18, 19, 26, 27]


def test_oracle_group_scale_order():
    """A group grid stores, per 128-row block, every group's 128 rows contiguously (block-major)."""
    s = np.arange(256 * 3, dtype=np.float32).reshape(256, 3)       # value = 3 * row + group
    stored = N.pack_scale(s).reshape(-1)
    assert stored[:4].tolist() == [0, 3, 24, 27]                    # block 0, group 0: rows 0, 1, 8, 9
    assert stored[128:132].tolist() == [1, 4, 25, 28]               # block 0, group 1
    assert stored[3 * 128:3 * 128 + 2].tolist() == [384, 387]       # block 1 (row 128), group 0


def test_oracle_weight_fragment_known_words():
    """With k = 128 (two 64-column tiles) the int32 words run: row 0 codes 0..7, row 0 codes 32..39 (the
    other k half of the 64-wide tile), row 8 codes 0..7 (the other row half of the 16-row pack), row 8
    codes 32..39, then row 0 codes 8..15 (next k lane) ...; 16 words on the next row lane (row 1, after
    the 4 k lanes x 2 x 2); 128 on the next 16-row pack (after 8 row lanes); 1024 on the next 64-column
    tile (after 8 packs)."""
    n, k = 128, 128
    codes = np.zeros((n, k), np.uint8)
    rng = np.random.default_rng(0)
    codes[:] = rng.integers(0, 16, (n, k))
    words = N.pack_weight(codes).view(np.uint32).reshape(-1)

    def word_of(row, c0):
        return sum(int(codes[row, c0 + t]) << (4 * t) for t in range(8))
    assert words[0] == word_of(0, 0)
    assert words[1] == word_of(0, 32)
    assert words[2] == word_of(8, 0)
    assert words[3] == word_of(8, 32)
    assert words[4] == word_of(0, 8)
    assert words[16] == word_of(1, 0)
    assert words[128] == word_of(16, 0)
    assert words[1024] == word_of(0, 64)


def test_oracle_lowrank_known_positions():
    """Stored position f of a 16 x 16 pack: f + 1 steps the k register (i_k + 1), f + 2 the k half
    (i_k + 8), f + 4 the n half (i_n + 8), f + 8 the k lane (i_k + 2), f + 32 the n lane (i_n + 1)."""
    w = np.arange(32 * 16, dtype=np.float32).reshape(32, 16)       # [in 32, rank 16], value = 16 in + r
    down = N.pack_lowrank(w, down=True).reshape(-1)                  # i_n = rank, i_k = input
    assert down[[0, 1, 2, 4, 8, 32]].tolist() == [w[0, 0], w[1, 0], w[8, 0], w[0, 8], w[2, 0], w[0, 1]]
    up = N.pack_lowrank(w, down=False).reshape(-1)                   # i_n = output, i_k = rank
    assert up[[0, 1, 2, 4, 8, 32]].tolist() == [w[0, 0], w[0, 1], w[0, 8], w[8, 0], w[0, 2], w[1, 0]]
    assert down[256] == w[16, 0]                                     # the next pack along the input


# ------------------------------------------------------------------ product decoders vs the oracle packers

@pytest.mark.parametrize("n,k", [(128, 128), (256, 384)])
def test_qweight_roundtrip(n, k):
    rng = np.random.default_rng(n + k)
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    stored = N.pack_weight(codes)
    assert np.array_equal(C.unpack_qweight(torch.from_numpy(stored), n, k).numpy(), codes)
    assert np.array_equal(C.pack_qweight(torch.from_numpy(codes)).numpy(), stored)


@pytest.mark.parametrize("n,g", [(128, 1), (256, 6), (384, 48)])
def test_group_scale_roundtrip(n, g):
    rng = np.random.default_rng(n * g)
    s = rng.uniform(1e-3, 1e-2, (n, g)).astype(np.float16)
    stored = N.pack_scale(s)
    assert np.array_equal(C.unpack_group_scales(torch.from_numpy(stored), n, 64 * g).numpy(), s)
    assert np.array_equal(C.pack_group_scales(torch.from_numpy(s)).numpy(), stored)


def test_vector_roundtrip():
    v = np.arange(3072, dtype=np.float32)
    stored = N.pack_scale(v.reshape(-1, 1)).reshape(-1)
    assert np.array_equal(C.unpack_vector(torch.from_numpy(stored), 3072).numpy(), v)
    assert np.array_equal(C.pack_vector(torch.from_numpy(v), 3072).numpy(), stored)


@pytest.mark.parametrize("down", [True, False])
def test_lowrank_roundtrip(down):
    rng = np.random.default_rng(int(down))
    w = rng.normal(size=(64, 32)).astype(np.float32)
    stored = N.pack_lowrank(w, down=down)
    assert np.array_equal(C.unpack_lowrank(torch.from_numpy(stored), down=down).numpy(), w)
    assert np.array_equal(C.pack_lowrank(torch.from_numpy(w), down=down).numpy(), stored)


def synthetic_int4_layer(n: int, k: int, rank: int, seed: int, *, second: str = ""):
    """Logical int4 svdq tensors and their stored (nunchaku) form, encoded by the oracle's packers."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    scales = rng.uniform(5e-4, 4e-3, (n, k // 64)).astype(np.float16)
    smooth = rng.uniform(0.5, 2.0, k).astype(np.float32)
    bias = rng.normal(0, 0.02, n).astype(np.float32)
    down = (rng.normal(0, 0.02, (k, rank))).astype(np.float32)
    up = (rng.normal(0, 0.02, (n, rank))).astype(np.float32)
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16)  # noqa: E731
    logical = dict(codes=codes, scales=scales, smooth=bf(smooth), bias=bf(bias), down=bf(down), up=bf(up))
    stored = {
        "qweight": torch.from_numpy(N.pack_weight(codes)),
        "wscales": torch.from_numpy(N.pack_scale(scales)),                      # fp16, the int4 lane's scale dtype
        "smooth_factor": torch.from_numpy(N.pack_scale(logical["smooth"].float().numpy().reshape(-1, 1))
                                          .reshape(-1)).to(torch.bfloat16),
        "bias": torch.from_numpy(N.pack_scale(logical["bias"].float().numpy().reshape(-1, 1)).reshape(-1))
        .to(torch.bfloat16),
        "proj_down": torch.from_numpy(N.pack_lowrank(logical["down"].float().numpy(), down=True)).to(torch.bfloat16),
        "proj_up": torch.from_numpy(N.pack_lowrank(logical["up"].float().numpy(), down=False)).to(torch.bfloat16),
    }
    if second == "channel":
        sc = rng.uniform(0.5, 2.0, n).astype(np.float32)
        logical["second"] = sc
        stored["wcscales"] = torch.from_numpy(N.pack_scale(sc.reshape(-1, 1)).reshape(-1))
    return logical, stored


def test_decode_linear_matches_logical():
    logical, stored = synthetic_int4_layer(256, 384, 32, seed=3, second="channel")
    dec = C.decode_int4_linear(stored, 256, 384)
    assert dec.rank == 32 and (dec.out_features, dec.in_features) == (256, 384)
    assert np.array_equal(dec.codes.numpy(), logical["codes"])
    assert np.array_equal(dec.scales.numpy(), logical["scales"]) and dec.scales.dtype == torch.float16
    assert torch.equal(dec.smooth_factor, logical["smooth"]) and torch.equal(dec.bias, logical["bias"])
    assert torch.equal(dec.proj_down, logical["down"]) and torch.equal(dec.proj_up, logical["up"])
    assert np.array_equal(dec.second.numpy(), logical["second"])


def test_decode_refusals():
    _, stored = synthetic_int4_layer(128, 128, 16, seed=4)
    with pytest.raises(C.SvdqLayoutError):
        C.decode_int4_linear({k: v for k, v in stored.items() if k != "proj_up"}, 128, 128)
    bad = dict(stored)
    bad["wscales"] = stored["wscales"].to(torch.float8_e4m3fn)       # the nvfp4 packaging's scale dtype
    with pytest.raises(C.SvdqLayoutError):
        C.decode_int4_linear(bad, 128, 128)
    bad = dict(stored)
    bad["wscales"] = (stored["wscales"].float() * (1 + 2 ** -12)).to(torch.float32)   # not representable in fp16
    with pytest.raises(C.SvdqLayoutError):
        C.decode_int4_linear(bad, 128, 128)
    with pytest.raises(C.SvdqLayoutError):
        C.decode_int4_linear(stored, 128, 256)                           # shapes disagree


def test_split_and_fold():
    logical, stored = synthetic_int4_layer(384, 256, 32, seed=5)
    dec = C.decode_int4_linear(stored, 384, 256)
    q, kk, v = C.split_decoded(dec, (128, 128, 128))
    assert torch.equal(kk.codes, dec.codes[128:256]) and torch.equal(v.proj_up, dec.proj_up[256:])
    assert kk.proj_down is dec.proj_down and kk.smooth_factor is dec.smooth_factor
    with pytest.raises(C.SvdqLayoutError):
        C.split_decoded(dec, (128, 128))
    # the dense fold equals deq(codes) * scale / smooth + up @ down^T (fp64 check on the logical tensors)
    lin = C.fold_decoded(dec, compute_dtype=torch.float32)
    c = logical["codes"].astype(np.int64)
    c = np.where(c >= 8, c - 16, c).astype(np.float64)
    w = (c.reshape(384, 4, 64) * logical["scales"].astype(np.float64)[..., None]).reshape(384, 256)
    w = w / logical["smooth"].double().numpy()[None, :] + logical["up"].double().numpy() @ logical["down"].double().numpy().T
    assert np.allclose(lin.weight.detach().double().numpy(), w, rtol=1e-6, atol=1e-8)


class _Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.to_q, self.to_k, self.to_v = nn.Linear(d, d), nn.Linear(d, d), nn.Linear(d, d)
        self.to_out = nn.ModuleList([nn.Linear(d, d)])


class _Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attn = _Attn(d)
        self.norm1 = nn.Module()
        self.norm1.linear = nn.Linear(d, 6 * d)


def test_plan_targets():
    m = nn.Module()
    m.blocks = nn.ModuleList([_Block(128)])
    assert C.plan_targets(m, "blocks.0.attn.to_out.0") == (("blocks.0.attn.to_out.0", 128),)
    assert C.plan_targets(m, "blocks.0.attn.to_qkv") == (("blocks.0.attn.to_q", 128), ("blocks.0.attn.to_k", 128),
                                                          ("blocks.0.attn.to_v", 128))
    with pytest.raises(C.SvdqLayoutError):
        C.plan_targets(m, "blocks.0.attn.to_nothing")
    with pytest.raises(C.SvdqLayoutError):
        C.plan_targets(m, "blocks.0.mlp.to_qkv")


def test_adanorm_split_table():
    assert C.adanorm_splits_for("QwenImageTransformer2DModel", "transformer_blocks.3.img_mod.1") == 6
    with pytest.raises(C.SvdqLayoutError):
        C.adanorm_splits_for("FluxTransformer2DModel", "transformer_blocks.0.norm1.linear")


def _skeleton(d):
    m = nn.Module()
    m.blocks = nn.ModuleList([_Block(d)])
    return m


def _decoded_qkv_and_out(d):
    _, qkv = synthetic_int4_layer(3 * d, d, 16, seed=21)
    _, out = synthetic_int4_layer(d, d, 16, seed=22)
    return {"blocks.0.attn.to_qkv": C.decode_int4_linear(qkv, 3 * d, d),
            "blocks.0.attn.to_out.0": C.decode_int4_linear(out, d, d)}


def test_swap_follows_the_dense_lane(monkeypatch):
    """The swap asks the process's qualified lane once; in the dense lane every linear becomes the folded
    bf16 Linear (the reference's dequant lane), with the fused projection split first."""
    from gen_worker_amd import qualify

    calls = []

    def fake_qualification():
        calls.append(1)
        return qualify.Qualification("dense", ["stubbed: int4 GEMM not profitable"])

    monkeypatch.setattr(qualify, "qualification", fake_qualification)
    d = 128
    model = _skeleton(d)
    decoded = _decoded_qkv_and_out(d)
    counts = C.swap_svdq_linears(model, decoded, device="cpu")
    assert counts == {"prefixes": 2, "linears": 4, "int4": 0, "blockwise": 0, "dense": 4, "lane": "dense",
                      "fp4_mode": "dense"}
    assert len(calls) == 1
    attn = model.blocks[0].attn
    for mod in (attn.to_q, attn.to_k, attn.to_v, attn.to_out[0]):
        assert type(mod) is nn.Linear and mod.weight.dtype == torch.bfloat16
    q_part = C.split_decoded(decoded["blocks.0.attn.to_qkv"], (d, d, d))[0]
    assert torch.equal(attn.to_q.weight, C.fold_decoded(q_part, device="cpu").weight)


def test_unavailable_lane_degrades_to_dense():
    """Without a GPU the int4 lane is unavailable: the lane resolves to dense instead of refusing."""
    from gen_worker_amd import qualify

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert qualify.resolve_lane() == "dense"
    assert qualify.resolve_lane("int4") == "int4"
    with pytest.raises(ValueError):
        qualify.resolve_lane("fp8")
    d = 128
    model = _skeleton(d)
    counts = C.swap_svdq_linears(model, _decoded_qkv_and_out(d), device="cpu")
    assert counts["lane"] == "dense" and counts["dense"] == 4


def test_swap_checks_the_whole_plan_before_changing_the_model():
    """A checkpoint linear whose shape does not fit its target is refused before any module is replaced."""
    d = 128
    model = _skeleton(d)
    decoded = _decoded_qkv_and_out(d)
    _, wide = synthetic_int4_layer(2 * d, d, 16, seed=23)
    decoded["blocks.0.norm1.linear"] = C.decode_int4_linear(wide, 2 * d, d)     # the model's Linear is [6d, d]
    before = {n: type(m) for n, m in model.named_modules()}
    with pytest.raises(C.SvdqLayoutError, match="norm1.linear"):
        C.swap_svdq_linears(model, decoded, device="cpu", lane="dense")
    assert {n: type(m) for n, m in model.named_modules()} == before


def test_adanorm_split_matches_whole_components():
    """The split table matches whole trailing path components, so a look-alike name is refused."""
    assert C.adanorm_splits_for("QwenImageTransformer2DModel", "img_mod.1") == 6
    with pytest.raises(C.SvdqLayoutError):
        C.adanorm_splits_for("QwenImageTransformer2DModel", "blocks.0.ximg_mod.1")
