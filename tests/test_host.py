"""CPU-side tests: the C-ABI library loads and exports its header, the golden
fixtures reproduce, and the host boundary refuses what it must (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import svdq_oracle as O

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = Path(__file__).resolve().parent / "golden"


def _header_symbols() -> list[str]:
    text = (ROOT / "include" / "gen_worker_amd.h").read_text()
    return sorted(set(re.findall(r"\b(gwa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    from gen_worker_amd import _native

    lib = _native.load()
    syms = _header_symbols()
    assert syms, "no symbols parsed from the header"
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(_native.EXPORTED_SYMBOLS)
    assert lib.gwa_version() == 1
    assert "gfx950" in _native.build_info()


def test_debug_build_exports_the_header_and_the_release_build_refuses_its_query():
    """The GWA_DEBUG build of the same sources exports the same header; only it answers
    gwa_debug_violations (the release library refuses before touching a device)."""
    import ctypes as C

    from gen_worker_amd import _native

    lib = _native.load()
    bits, first = C.c_uint32(7), C.c_uint64(7)
    assert lib.gwa_debug_violations(C.byref(bits), C.byref(first), 0) == 1
    assert "not a debug build" in lib.gwa_last_error().decode()
    if not _native.debug_library_path().exists():
        pytest.skip("the debug library is not built (`python -m gen_worker_amd.build` builds it)")
    dbg = _native.load_debug()
    for s in _header_symbols():
        assert hasattr(dbg, s), s
    assert "debug" in dbg.gwa_build_info().decode()


def test_library_is_a_gfx950_code_object():
    from gen_worker_amd import _native

    data = _native.library_path().read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_fp6_tile_model_choices():
    """The tile model (host code only): 288-row tiles for 4608-token layers (one tile per CU at N=3072),
    256 x 192 for 4096 tokens, 256 x 128 at 512 tokens and wide outputs, the 64 x 128 tile (two to a CU) for
    short inputs, the forced tile while one is set."""
    from gen_worker_amd import _native

    lib = _native.load()
    tile = lib.gwa_svdq_gemm_w4a4_fp6_tile
    assert tile(0, 3072) == -1 and tile(16, 0) == -1
    assert tile(4608, 3072) == 4 and tile(4608, 9216) == 4
    assert tile(4096, 3072) == 5
    assert tile(512, 9216) == 1 and tile(512, 12288) == 1
    # 96 / 192 / 384 64 x 128 tiles against 48 / 96 / 192 128 x 128 ones (15.5 vs 21.8 us measured at 256)
    assert tile(256, 3072) == 6 and tile(512, 3072) == 6 and tile(1024, 3072) == 6
    assert tile(256, 9216) == 6 and tile(256, 12288) == 6
    prev = lib.gwa_svdq_gemm_w4a4_fp6_force_tile(1)
    try:
        assert tile(4608, 3072) == 1
    finally:
        lib.gwa_svdq_gemm_w4a4_fp6_force_tile(prev)
    assert tile(4608, 3072) == 4


def test_w8a8_tile_choice():
    """The W8A8 GEMM's tile choice (host code only): 256 x 256 when its rounds over the 256 CUs (2.7 times a
    128 x 128 round each) take less time than the 128 x 128 grid's (QKV, 4096^3, config 1's 216 tiles, QKV at
    M=1024), 128 x 128 for small grids, for K % 128 != 0 and for K >= 2^23; the forced tile while one is set."""
    from gen_worker_amd import _native

    lib = _native.load()
    tile = lib.gwa_w8a8_gemm_tile
    assert tile(0, 3072, 3072) == -1 and tile(16, 0, 128) == -1
    assert tile(4608, 9216, 3072) == 1 and tile(4096, 4096, 4096) == 1 and tile(4608, 3072, 3072) == 1
    assert tile(16384, 9216, 3072) == 1
    assert tile(1024, 9216, 3072) == 1  # 144 tiles in one round against three rounds of 576
    assert tile(256, 9216, 3072) == 0 and tile(1024, 3072, 3072) == 0
    assert tile(4608, 9216, 3136) == 0 and tile(4608, 9216, 1 << 23) == 0
    prev = lib.gwa_w8a8_gemm_force_tile(0)
    try:
        assert tile(4608, 9216, 3072) == 0
        lib.gwa_w8a8_gemm_force_tile(1)
        assert tile(256, 9216, 3072) == 1 and tile(4608, 9216, 3136) == 0
    finally:
        lib.gwa_w8a8_gemm_force_tile(prev)
    assert tile(4608, 9216, 3072) == 1


def test_invalid_arguments_are_refused_before_any_launch():
    from gen_worker_amd import _native

    lib = _native.load()
    # K not a multiple of 64: validated on the host, no device touched
    rc = lib.gwa_svdq_quant_int4(None, 100, None, None, None, 0, 0, None, None, None, 4, 100, None)
    assert rc == 1 and "multiple of 64" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_quant_int4(None, 64, None, None, None, 0, 7, None, None, None, 4, 64, None)
    assert rc == 1 and "out_format" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_quant_int4(None, 192, None, None, None, 0, 1, None, None, None, 4, 192, None)
    assert rc == 1 and "gwa_svdq_quant_fp6" in lib.gwa_last_error().decode()
    # the fp6 records take any K % 64 == 0 (K % 128 == 64 ends in a half stage)
    rc = lib.gwa_svdq_quant_fp6(None, 160, None, None, None, 0, None, None, 4, 160, None)
    assert rc == 1 and "multiple of 64" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_quant_fp6(None, 192, None, None, None, 0, None, None, 4, 192, None)
    assert rc == 1 and "null pointer" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_prep_proj_down_fp6(None, None, 160, 32, None)
    assert rc == 1 and "multiple of 64" in lib.gwa_last_error().decode()
    assert lib.gwa_svdq_quant_fp6_partials(77, 320, 32) == 3 and lib.gwa_svdq_quant_fp6_partials(77, 160, 32) == 0
    rc = lib.gwa_svdq_la_reduce(None, 0, 4, 32, None, None)
    assert rc == 1 and "bad shape" in lib.gwa_last_error().decode()
    # partial-slot counts: kernel 1 splits K=3072 of 4608 rows over 6 ranges; the 256-wide GEMM tiles of
    # N = 12288 give 48 column tiles, the 128-wide tiles of a small M twice as many per N
    assert lib.gwa_svdq_quant_fp6_partials(4608, 3072, 32) == 6
    assert lib.gwa_svdq_gemm_w4a4_fp6_next_partials(4608, 12288) == 48
    assert lib.gwa_svdq_gemm_w4a4_fp6_next_partials(256, 3072) == 24
    assert lib.gwa_svdq_quant_fp6_partials(4608, 3072, 0) == 0
    rc = lib.gwa_svdq_gemm_w4a4_fp6(None, 0, None, 0, None, None, 0, None, None, 0, None, None, 0, 0, 8, 64, 160,
                                    None)
    assert rc == 1 and "multiple of 64" in lib.gwa_last_error().decode()
    # K = 192: two stages (the second a half stage), so the records and their slack are 2 * 8 * 104 + 1024 bytes
    rc = lib.gwa_svdq_gemm_w4a4_fp6(None, 2 * 8 * 104, None, 0, None, None, 0, None, None, 0, None, None, 0, 0, 8,
                                    64, 192, None)
    assert rc == 1 and "null pointer" in lib.gwa_last_error().decode()
    assert lib.gwa_svdq_w4a4_linear_fp6_workspace(8, 192, 32) > 0 == lib.gwa_svdq_w4a4_linear_fp6_workspace(8, 160, 32)
    # the next-layer epilogue needs whole 128-column stages and a record buffer
    rc = lib.gwa_svdq_gemm_w4a4_fp6_next(None, 0, None, 0, None, None, 0, None, None, 0, None, None, 0, None, None,
                                         0, None, None, 8, 192, 128, None)
    assert rc == 1 and "multiple of 128" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_gemm_w4a4_fp6_next(None, 0, None, 0, None, None, 0, None, None, 0, None, None, 0, None, None,
                                         0, None, None, 8, 256, 128, None)
    assert rc == 1 and "next_q6" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_prep_proj_down(None, None, 64, 24, None)
    assert rc == 1 and "rank" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_gemm_w4a4(None, None, None, None, None, None, 0, None, None, 0, None, None, 0, 0,
                                8, 24, 128, None)
    assert rc == 1 and "multiple of 16" in lib.gwa_last_error().decode()
    rc = lib.gwa_w8a8_gemm(None, None, None, 8, None, None, 0, None, 7, 8, 64, 64, None)
    assert rc == 1 and "out_dtype" in lib.gwa_last_error().decode()
    rc = lib.gwa_transpose_2d(None, None, 4, 4, 3, None)
    assert rc == 1
    # empty problems are no-ops
    assert lib.gwa_svdq_quant_int4(None, 64, None, None, None, 0, 0, None, None, None, 0, 64, None) == 0
    assert lib.gwa_probe_add_one(None, None, 0, None) == 0


def test_record_buffer_sizes_are_checked_at_the_c_abi():
    """Every C entry point that reads fp6 records takes each record pointer's readable byte count and refuses a
    buffer shorter than the records plus GWA_FP6_RECORD_SLACK (the GEMMs' 1 KB copy runs may read that far past
    the last record) with GWA_ERR_INVALID before anything is enqueued; the psums kernel reads through
    range-checked lane offsets and needs the records only. The pointers below are never dereferenced: every
    call is refused on its sizes before any HIP call."""
    from gen_worker_amd import _native as nat

    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)   # aligned, non-null; never touched
    m, n, k = 288, 192, 384
    qa_need, qw_need, slack = (k // 128) * m * nat.FP6_REC, (k // 128) * n * nat.FP6_REC, 1024
    for fn in ("gwa_svdq_gemm_w4a4_fp6", "gwa_svdq_gemm_w4a4_fp6_next"):
        def call(qa_b, qw_b):
            if fn == "gwa_svdq_gemm_w4a4_fp6":
                return lib.gwa_svdq_gemm_w4a4_fp6(fake, qa_b, fake, qw_b, None, None, 0, None, None, 0, None, fake,
                                                  0, 0, m, n, k, None)
            return lib.gwa_svdq_gemm_w4a4_fp6_next(fake, qa_b, fake, qw_b, None, None, 0, None, None, 0, None, fake,
                                                   0, None, None, 0, fake, None, m, 256, k, None)
        nn_ = n if fn == "gwa_svdq_gemm_w4a4_fp6" else 256
        qwn = (k // 128) * nn_ * nat.FP6_REC
        assert call(qa_need + slack - 1, qwn + slack) == 1
        assert "qa6 has" in lib.gwa_last_error().decode() and "slack" in lib.gwa_last_error().decode()
        assert call(qa_need + slack, qwn + slack - 1) == 1
        assert "qw6 has" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_group_psums_fp6(fake, qa_need - 1, fake, qw_need, fake, m, n, k, None)
    assert rc == 1 and "record buffers" in lib.gwa_last_error().decode()
    rc = lib.gwa_svdq_group_psums_fp6(fake, qa_need, fake, qw_need - 1, fake, m, n, k, None)
    assert rc == 1 and "record buffers" in lib.gwa_last_error().decode()
    for fn in ("gwa_svdq_w4a4_linear_fp6", "gwa_svdq_w4a4_linear_fp6_noalloc"):
        tail = (fake, 1 << 30, None) if fn == "gwa_svdq_w4a4_linear_fp6" else (None,)
        rc = getattr(lib, fn)(fake, k, None, None, None, 0, fake, qw_need + slack - 1, None, 0, None, None, fake, 0,
                              0, m, n, k, *tail)
        assert rc == 1 and "qw6 has" in lib.gwa_last_error().decode(), lib.gwa_last_error()


def test_native_error_is_raised_with_message():
    from gen_worker_amd import _native

    with pytest.raises(_native.NativeError, match="multiple of 64"):
        _native.call("gwa_w8a8_gemm", None, None, None, 8, None, None, 0, None, 0, 8, 64, 100, None)


def test_ops_refuse_cpu_tensors():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd.ops import SvdqOpError

    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises(SvdqOpError, match="GPU only"):
        torch.ops.cozy_gen_worker.svdq_quant(x, None, torch.ones(()), False)
    with pytest.raises(SvdqOpError, match="blocked"):
        torch.ops.cozy_gen_worker.svdq_quant(x, None, torch.ones(()), True)
    with pytest.raises(SvdqOpError, match="GPU only"):
        torch.ops.cozy_gen_worker.w8a8_quant(x)


def test_fake_impls_trace_shapes():
    import gen_worker_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(77, 384, dtype=torch.bfloat16)
        pdo = torch.ops.cozy_gen_worker.svdq_prep_proj_down(torch.empty(384, 32, dtype=torch.bfloat16))
        assert pdo.shape == (512, 32)
        q, s, la = torch.ops.cozy_gen_worker.svdq_quant_lora(x, None, None, pdo)
        q6, la6 = torch.ops.cozy_gen_worker.svdq_quant_fp6(x, None, None, None)
        assert q6.shape == (3, 77, 104) and la6.shape == (77, 0)
        pdo6 = torch.ops.cozy_gen_worker.svdq_prep_proj_down_fp6(torch.empty(384, 32, dtype=torch.bfloat16))
        q6b, la6b = torch.ops.cozy_gen_worker.svdq_quant_fp6(x, None, None, pdo6)
        assert pdo6.shape == (384, 32) and la6b.shape == (77, 32) and la6b.dtype == torch.bfloat16
        w6 = torch.ops.cozy_gen_worker.svdq_pack_weight_fp6(torch.empty(128, 192, dtype=torch.uint8),
                                                           torch.empty(128, 6, dtype=torch.float16))
        assert w6.shape == (3, 128, 104)
        # K = 320 (K % 128 == 64): records of 3 stages, the last a half stage; proj_down rows padded to 384
        xh = torch.empty(77, 320, dtype=torch.bfloat16)
        pdoh = torch.ops.cozy_gen_worker.svdq_prep_proj_down_fp6(torch.empty(320, 32, dtype=torch.bfloat16))
        qh, lah = torch.ops.cozy_gen_worker.svdq_quant_fp6(xh, None, None, pdoh)
        wh = torch.ops.cozy_gen_worker.svdq_pack_weight_fp6(torch.empty(128, 160, dtype=torch.uint8),
                                                           torch.empty(128, 5, dtype=torch.float16))
        assert pdoh.shape == (384, 32) and qh.shape == (3, 77, 104) and lah.shape == (77, 32)
        assert wh.shape == (3, 128, 104)
        y6 = torch.ops.cozy_gen_worker.svdq_w4a4_linear_fp6(q6, w6, None, None, None, None, None, torch.bfloat16,
                                                            False)
        assert y6.shape == (77, 128) and y6.dtype == torch.bfloat16
        assert torch.ops.cozy_gen_worker.svdq_group_psums_fp6(q6, w6).shape == (77, 128, 6)
        nq = torch.empty(4, 77, 104, dtype=torch.uint8)
        yn = torch.ops.cozy_gen_worker.svdq_w4a4_linear_fp6_next(q6, w6, None, None, None, None, None, True, None,
                                                                 None, nq, None, 3, True)
        assert yn.shape == (77, 128) and yn.dtype == torch.bfloat16
        yn0 = torch.ops.cozy_gen_worker.svdq_w4a4_linear_fp6_next(q6, w6, None, None, None, None, None, False,
                                                                  None, None, nq, None, 0, False)
        assert yn0.shape == (77, 0)
        assert torch.ops.cozy_gen_worker.svdq_quant_fp6_into(x, None, None, nq, None) is None
        la_r = torch.ops.cozy_gen_worker.svdq_la_reduce(torch.empty(3, 77, 32))
        assert la_r.shape == (77, 32) and la_r.dtype == torch.bfloat16
        assert q.shape == (77, 192) and s.shape == (77, 6) and la.shape == (77, 32)
        w = torch.empty(128, 192, dtype=torch.uint8)
        ws = torch.empty(128, 6, dtype=torch.float16)
        y = torch.ops.cozy_gen_worker.svdq_w4a4_linear(q, s, w, ws, None, None, la, torch.empty(128, 32,
                                                       dtype=torch.bfloat16), None, torch.float16, False)
        assert y.shape == (77, 128) and y.dtype == torch.float16


def test_concat_halves_refuse_outside_the_fused_contract():
    """SvdqConcat (the two halves of the single block's proj_out-over-[attention, MLP] forward) takes only the
    fp6 lane's fused contract: modules off the GPU, or widths that do not meet, are refused before any launch."""
    from gen_worker_amd import SvdqFusedError, SvdqW4A4Linear
    from gen_worker_amd.svdq import SvdqConcat

    mlp = SvdqW4A4Linear(256, 512, rank=32, bias=True, activation="gelu_tanh")
    proj = SvdqW4A4Linear(256 + 512, 256, rank=32, bias=True)
    n = torch.zeros(4, 256, dtype=torch.bfloat16)
    with pytest.raises(SvdqFusedError, match="fused contract"):
        SvdqConcat(proj, mlp, n, 256)          # CPU modules: not the fp6 lane
    with pytest.raises(SvdqFusedError, match="fused contract"):
        SvdqConcat(proj, mlp, n, 128)          # 128 + 512 != 768


def test_capture_graph_keeps_the_cyclic_collector_off_only_while_capturing(monkeypatch):
    """graphs.capture_graph collects garbage first, runs the capture with Python's cyclic collector off, and
    restores it afterwards, also when the captured function raises (CUDA calls stubbed)."""
    import contextlib
    import gc

    from gen_worker_amd import graphs

    class _Stream:
        def wait_stream(self, other):
            pass

    seen = []
    monkeypatch.setattr(torch.cuda, "Stream", lambda *a, **k: _Stream())
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a, **k: _Stream())
    monkeypatch.setattr(torch.cuda, "CUDAGraph", lambda *a, **k: object())
    monkeypatch.setattr(torch.cuda, "stream", lambda s: contextlib.nullcontext())
    monkeypatch.setattr(torch.cuda, "graph", lambda g, stream=None: contextlib.nullcontext())
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    assert gc.isenabled()
    g, out = graphs.capture_graph(lambda: seen.append(gc.isenabled()) or 7)
    assert out == 7 and seen == [False] and gc.isenabled()

    def boom():
        seen.append(gc.isenabled())
        raise RuntimeError("capture failed")

    with pytest.raises(RuntimeError, match="capture failed"):
        graphs.capture_graph(boom)
    assert seen == [False, False] and gc.isenabled()
    gc.disable()
    try:  # a caller that runs with the collector off keeps it off
        graphs.capture_graph(lambda: None)
        assert not gc.isenabled()
    finally:
        gc.enable()


def test_module_tracks_in_place_updates_of_its_primary_buffers():
    """The derived buffers are rebuilt on the next forward after ``weight`` / ``weight_scale`` / ``proj_down``
    change in place (version counter) or are reassigned (identity); nothing else triggers a rebuild, and tensors
    made under inference mode (no version counter) are tracked by identity without raising."""
    from gen_worker_amd import SvdqW4A4Linear

    m = SvdqW4A4Linear(128, 128, rank=0, bias=False, device="cpu")
    calls = []
    orig = m.refresh_derived
    m.refresh_derived = lambda: (calls.append(1), orig())[1]
    m._ensure_derived()
    m._ensure_derived()
    assert len(calls) == 1, "an unchanged module rebuilt its derived buffers"
    with torch.no_grad():
        m.weight.add_(1)
    m._ensure_derived()
    assert len(calls) == 2, "an in-place weight update was missed"
    with torch.no_grad():
        m.weight_scale.mul_(2)
    m._ensure_derived()
    assert len(calls) == 3, "an in-place weight_scale update was missed"
    m.weight = torch.zeros_like(m.weight)
    m._ensure_derived()
    m._ensure_derived()
    assert len(calls) == 4, "a reassigned weight was missed (or rebuilt twice)"
    m.second.fill_(3.0)  # read by the kernels directly, nothing derived from it
    m._ensure_derived()
    assert len(calls) == 4
    with torch.inference_mode():
        mi = SvdqW4A4Linear(128, 128, rank=16, bias=False, device="cpu")
        v = mi._primary_versions()
    assert all(e is not None and e[1] is None for e in v), v


def test_module_contract_refusals():
    from gen_worker_amd import SvdqFusedError, SvdqW4A4Linear, W8a8Error, Int8ScaledLinear

    with pytest.raises(SvdqFusedError):
        SvdqW4A4Linear(100, 128, rank=32, bias=True)
    with pytest.raises(SvdqFusedError):
        SvdqW4A4Linear(128, 120, rank=32, bias=True)
    with pytest.raises(SvdqFusedError):
        SvdqW4A4Linear(128, 128, rank=24, bias=True)
    with pytest.raises(W8a8Error):
        Int8ScaledLinear(100, 128, bias=False)
    m = SvdqW4A4Linear(3072, 3072, rank=32, bias=True)
    assert m.weight.shape == (3072, 1536) and m.weight.dtype == torch.uint8
    assert m.weight_scale.shape == (3072, 48) and m.weight_scale.dtype == torch.float16
    assert m.proj_down.shape == (3072, 32) and m.proj_up.shape == (3072, 32)
    names = set(dict(m.named_buffers()))
    assert {"weight", "weight_scale", "second", "smooth_factor", "proj_down", "proj_up"} <= names


def test_fold_to_dense_module_matches_oracle():
    """The any-hardware fallback lane of the module equals the oracle's folded weight."""
    from gen_worker_amd import synthetic
    from gen_worker_amd.svdq import build_svdq_w4a4_linear, fold_to_dense

    L = synthetic.w4a4_layer(128, 256, 16)
    mod = build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                 proj_up=L.proj_up, bias=L.bias, device="cpu")
    lin = fold_to_dense(mod, compute_dtype=torch.float32)
    b = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    want = O.fold_to_dense(L.qweight.numpy(), L.wscales.numpy(), b(L.smooth), b(L.proj_down), b(L.proj_up))
    assert np.allclose(lin.weight.detach().numpy(), want, rtol=1e-6, atol=1e-7)


def test_svdquant_decompose_reconstructs():
    from gen_worker_amd.svdq import svdquant_decompose

    g = torch.Generator().manual_seed(0)
    w = torch.randn(64, 128, generator=g)
    sm = torch.rand(128, generator=g) + 0.5
    res, down, up = svdquant_decompose(w, sm, 16)
    back = res / sm.reshape(1, -1) + up @ down.t()
    assert torch.allclose(back, w, atol=1e-4)


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("*.npz")))
def test_golden_fixtures_reproduce(name):
    """The pinned oracle regenerates every committed fixture bit for bit."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    import tempfile

    with tempfile.TemporaryDirectory() as d:
        mg.make(Path(d))
        a = np.load(GOLDEN / name)
        b = np.load(Path(d) / name)
        assert set(a.files) == set(b.files)
        for f in a.files:
            assert np.array_equal(a[f], b[f]), f


def test_synthetic_inputs_are_deterministic():
    from gen_worker_amd import synthetic

    a = synthetic.activation(8, 3072, outlier_frac=0.005, outlier_scale=30.0)
    b = synthetic.activation(8, 3072, outlier_frac=0.005, outlier_scale=30.0)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert int((a.float().abs().amax(dim=0) > 20).sum()) > 0
    s = synthetic.smooth_factor(3072)
    assert float(s.float().min()) >= 0.25 and float(s.float().max()) <= 4.0


def test_qualification_torch_chains_match_oracle():
    """The qualification gates' torch chains (the quantizer the kernels must equal byte for byte, the int4
    packer, the fp6 record decoder) against the oracle on the CPU."""
    import numpy as np

    from helpers import bits16
    from oracle import svdq_oracle as O

    from gen_worker_amd import qualify

    g = torch.Generator().manual_seed(5)
    for m, k, smooth in ((33, 256, True), (7, 640, False), (64, 3072, True)):
        x = (torch.randn(m, k, generator=g) * 3).to(torch.bfloat16)
        x[0, :64] = 0.0                                   # a zero group
        x[1, 5] = 1000.0                                  # an outlier
        sm = (torch.rand(k, generator=g) * 3.75 + 0.25).to(torch.bfloat16) if smooth else None
        q, s = qualify.quantize_act_torch(x, sm)
        wq, ws = O.quantize_act_int4(bits16(x), bits16(sm) if smooth else None)
        assert np.array_equal(qualify.pack_int4_torch(q).numpy(), wq)
        assert np.array_equal(s.view(torch.int16).numpy().view(np.uint16), ws.view(np.uint16))
    # fp6 records: encode known codes (element t of a group at bits 6t of the group's 48 bytes)
    e3m2 = {0: 0x00, 1: 0x0C, 2: 0x10, 3: 0x12, 4: 0x14, 5: 0x15, 6: 0x16, 7: 0x17}
    rng = np.random.default_rng(0)
    S, M = 3, 5
    codes = rng.integers(-8, 8, size=(M, 128 * S))
    scales = rng.standard_normal((M, 2 * S)).astype(np.float16)
    rec = np.zeros((S, M, 104), np.uint8)
    for st in range(S):
        for r in range(M):
            for gi in range(2):
                bits = 0
                for t in range(64):
                    c = int(codes[r, 128 * st + 64 * gi + t])
                    v = (0x20 | (0x18 if c == -8 else e3m2[-c])) if c < 0 else e3m2[c]
                    bits |= v << (6 * t)
                rec[st, r, 48 * gi:48 * gi + 48] = np.frombuffer(bits.to_bytes(48, "little"), np.uint8)
            rec[st, r, 96:100] = np.frombuffer(scales[r, 2 * st:2 * st + 2].tobytes(), np.uint8)
    dc, ds = qualify.decode_fp6_records_torch(torch.from_numpy(rec))
    assert np.array_equal(dc.numpy(), codes.astype(np.int8))
    assert np.array_equal(ds.numpy().view(np.uint16), scales.view(np.uint16))


def test_qualification_without_gpu_is_unavailable():
    from gen_worker_amd import qualify

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    q = qualify.qualify()
    assert q.lane == "unavailable" and q.reasons


def test_record_slack_helpers_on_cpu_tensors():
    """The slack the fp6 GEMM needs past a record tensor is measured on its storage, views included."""
    from gen_worker_amd import ops

    n = 3 * 5 * 104
    full = torch.empty(n + ops.RECORD_SLACK, dtype=torch.uint8)
    rec = full[:n].view(3, 5, 104)
    assert ops.record_slack_bytes(rec) == ops.RECORD_SLACK
    ops._check_record_slack("t", rec, "rec")
    inner = full[104:104 + 2 * 104].view(1, 2, 104)          # a view deep inside the storage
    assert ops.record_slack_bytes(inner) == n + ops.RECORD_SLACK - 3 * 104
    bare = rec.clone()
    assert ops.record_slack_bytes(bare) == 0
    with pytest.raises(ops.SvdqOpError, match="records_empty"):
        ops._check_record_slack("t", bare, "rec")


def test_module_move_drops_derived_buffers():
    """Moves and casts drop the derived operand-order buffers (rebuilt with slack on the next GPU forward)."""
    from gen_worker_amd.svdq import SvdqW4A4Linear

    mod = SvdqW4A4Linear(256, 128, rank=16, bias=True, device="cpu")
    mod.weight_fp6 = torch.zeros(2, 128, 104, dtype=torch.uint8)
    mod.proj_down_op6 = torch.zeros(256, 16, dtype=torch.bfloat16)
    mod.proj_down_op = torch.zeros(256, 16, dtype=torch.bfloat16)
    mod = mod.to("cpu")
    assert mod.weight_fp6 is None and mod.proj_down_op6 is None and mod.proj_down_op is None
    assert mod.weight.shape == (128, 128) and mod.proj_down.shape == (256, 16)


def test_w8a8_module_modes_on_cpu():
    """Int8ScaledLinear's mode contract, host side: the reference's two GEMM modes only, an ``input_scale``
    state-dict entry exactly when the layer has a static scale, and a static scale must be one scalar."""
    from gen_worker_amd import synthetic
    from gen_worker_amd.w8a8 import Int8ScaledLinear, W8a8Error, build_int8_linear

    with pytest.raises(W8a8Error, match="gemm_mode"):
        Int8ScaledLinear(64, 64, bias=False, gemm_mode="blockwise")
    assert "input_scale" not in Int8ScaledLinear(64, 64, bias=False).state_dict()
    sd = Int8ScaledLinear(64, 64, bias=False, static_input_scale=True, gemm_mode="pertensor").state_dict()
    assert sd["input_scale"].shape == (1, 1) and sd["input_scale"].dtype == torch.float32
    L = synthetic.w8a8_layer(64, 64)
    mod = build_int8_linear(qweight=L.qweight, weight_scale=L.weight_scale, bias=None, device="cpu",
                            input_scale=torch.tensor(0.5), gemm_mode="pertensor")
    assert float(mod.input_scale) == 0.5 and mod.gemm_mode == "pertensor"
    with pytest.raises(W8a8Error, match="one scalar"):
        build_int8_linear(qweight=L.qweight, weight_scale=L.weight_scale, bias=None, device="cpu",
                          input_scale=torch.ones(2))


def test_dit_glue_refuses_bad_shapes_before_any_launch():
    """The DiT block glue entry points validate on the host (no device touched)."""
    from gen_worker_amd import _native

    lib = _native.load()
    rc = lib.gwa_dit_qk_norm_rope(None, None, None, 64 * 2, None, None, None, None, 0, 8, None, None, None,
                                  64 * 2, 4, 2, 64, 1e-6, None)
    assert rc == 1 and "head_dim" in lib.gwa_last_error().decode()
    rc = lib.gwa_dit_qk_norm_rope(None, None, None, 256, None, None, None, None, 6, 8, None, None, None, 256, 4,
                                  2, 128, 1e-6, None)
    assert rc == 1 and "outside" in lib.gwa_last_error().decode()
    rc = lib.gwa_dit_adaln_modulate(None, 640, None, None, None, 640, 4, 640, 1e-6, None)
    assert rc == 1 and "multiple of 512" in lib.gwa_last_error().decode()
    rc = lib.gwa_dit_gate_residual(None, 12, None, 12, None, None, 12, 4, 12, None)
    assert rc == 1 and "multiple of 8" in lib.gwa_last_error().decode()
    # empty problems are no-ops
    assert lib.gwa_dit_adaln_modulate(None, 512, None, None, None, 512, 0, 512, 1e-6, None) == 0
    assert lib.gwa_dit_gate_residual(None, 8, None, 8, None, None, 8, 0, 8, None) == 0


def test_bench_dit_child_results_and_failures_map_to_the_line(monkeypatch):
    """bench.run_dit_child: the child's --workload dit line becomes the default line's dit_* keys; a child
    that fails, prints an unreadable line or runs too long leaves only dit_error (the config-1 figures stand)."""
    import argparse
    import importlib.util
    import json
    import subprocess
    import types

    spec = importlib.util.spec_from_file_location("bench_under_test", Path(__file__).resolve().parents[1] / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    args = argparse.Namespace(dit_steps=3, modulation="w4a4")
    good = {"value": 72.5, "bf16_gemm_ms": 96.0, "speedup_vs_bf16": 1.3241,
            "config": {"lane": "int4", "gate_lane": "int4"}, "outputs_finite": {"w4a4": True, "bf16": True}}
    calls = []

    def fake(stdout, rc=0, exc=None):
        def run(cmd, **kw):
            calls.append(cmd)
            if exc is not None:
                raise exc
            return types.SimpleNamespace(returncode=rc, stdout=stdout)
        return run

    monkeypatch.setattr(subprocess, "run", fake("progress\n" + json.dumps(good) + "\n"))
    out = bench.run_dit_child(args)
    assert out["dit_step_ms"] == 72.5 and out["dit_bf16_step_ms"] == 96.0 and out["dit_lane"] == "int4"
    assert out["dit_outputs_finite"] is True and "dit_error" not in out
    assert calls[-1][2:] == [str(Path(bench.__file__).resolve()), "--workload", "dit", "--steps", "3", "--warmup",
                             "1", "--modulation", "w4a4", "--attention", "sdpa"]
    for run in (fake(json.dumps(good), rc=134), fake("no line"), fake('{"value": 1.0}'), fake("{not json"),
                fake("", exc=subprocess.TimeoutExpired(cmd="x", timeout=900))):
        monkeypatch.setattr(subprocess, "run", run)
        out = bench.run_dit_child(args)
        assert set(out) == {"dit_error"}, out
