"""GPU tests of the debug build (``libgen_worker_amd_debug.so``, compiled with GWA_DEBUG).

Its kernels check the global accesses the hardware does not range-check (the fp6 GEMMs' 1 KB record copies at
scalar offsets, which may reach GWA_FP6_RECORD_SLACK past the records) and the stores whose silent drop would
hide a mistake (kernel 1's records, the GEMMs' outputs, the W8A8 copies' K offsets), and record a failed check
instead of making the access. On in-contract calls across ragged shapes and every forced tile, no check may
fail, and every output must equal the release library's bit for bit (the checks change no arithmetic).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def libs():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native

    rel = _native.load()
    if not _native.debug_library_path().exists():
        pytest.skip("the debug library is not built (`python -m gen_worker_amd.build` builds it)")
    dbg = _native.load_debug()
    assert "debug" in dbg.gwa_build_info().decode()
    yield rel, dbg


def _violations(lib, clear=True):
    bits, first = ctypes.c_uint32(0), ctypes.c_uint64(0)
    assert lib.gwa_debug_violations(ctypes.byref(bits), ctypes.byref(first), int(clear)) == 0, \
        lib.gwa_last_error()
    return bits.value, first.value


def _ok(rc, lib):
    assert rc == 0, lib.gwa_last_error().decode()


def _quant(lib, x, m, k, rank, pdo, smooth):
    """kernel 1 into records (with 1 KB of slack) + partial slots, then the reduce: (records, la)."""
    from gen_worker_amd import ops

    q6 = ops.records_empty(ops.fp6_stages(k), m, torch.device(DEV))
    p = int(lib.gwa_svdq_quant_fp6_partials(m, k, rank)) if rank else 0
    part = torch.empty(max(p, 1), m, max(rank, 1), dtype=torch.float32, device=DEV)
    la = torch.empty(m, max(rank, 1), dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    _ok(lib.gwa_svdq_quant_fp6(x.data_ptr(), k, smooth.data_ptr(), None, pdo.data_ptr() if rank else None, rank,
                               q6.data_ptr(), part.data_ptr() if rank else None, m, k, s), lib)
    if rank:
        _ok(lib.gwa_svdq_la_reduce(part.data_ptr(), p, m, rank, la.data_ptr(), s), lib)
    return q6, la


_SHAPES = [(1, 48, 128, 16), (77, 256, 512, 32), (289, 208, 384, 32), (600, 1040, 640, 0), (1100, 3072, 1280, 64),
           (45, 256, 320, 32), (300, 96, 64, 16)]   # the last two end in a half stage (K % 128 == 64)


@pytest.mark.parametrize("m,n,k,rank", _SHAPES)
def test_debug_build_fp6_lane_no_violation_and_identical(libs, m, n, k, rank):
    from gen_worker_amd import ops, synthetic
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    rel, dbg = libs
    _violations(dbg)
    layer = synthetic.w4a4_layer(n, k, rank or 16)
    mod = build_svdq_w4a4_linear(qweight=layer.qweight, wscales=layer.wscales, smooth=layer.smooth,
                                 proj_down=layer.proj_down, proj_up=layer.proj_up, bias=layer.bias,
                                 device=torch.device(DEV))
    mod._ensure_derived()
    x = synthetic.activation(m, k, outlier_frac=0.01, outlier_scale=20.0).to(DEV)
    pdo, up = mod.proj_down_op6, mod.proj_up
    outs = {}
    for name, lib in (("rel", rel), ("dbg", dbg)):
        q6, la = _quant(lib, x, m, k, rank, pdo, mod.smooth_factor)
        res = [q6.clone()] + ([la.clone()] if rank else [])  # rank 0: la is never written
        for tile in range(7):  # every fp6 GEMM tile (the 288- and 256-row pipelined ones included)
            lib.gwa_svdq_gemm_w4a4_fp6_force_tile(tile)
            out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
            _ok(lib.gwa_svdq_gemm_w4a4_fp6(q6.data_ptr(), ops.readable_bytes(q6), mod.weight_fp6.data_ptr(),
                                           ops.readable_bytes(mod.weight_fp6), None, mod.second.data_ptr(),
                                           mod.second.numel(), la.data_ptr() if rank else None,
                                           up.data_ptr() if rank else None, rank, mod.bias.data_ptr(),
                                           out.data_ptr(), 0, 0, m, n, k, torch.cuda.current_stream().cuda_stream),
                lib)
            res.append(out)
        lib.gwa_svdq_gemm_w4a4_fp6_force_tile(-1)
        torch.cuda.synchronize()
        outs[name] = res
    bits, first = _violations(dbg)
    assert bits == 0, f"debug checks failed: sites {bits:#x}, first {first:#x}"
    for a, b in zip(outs["rel"], outs["dbg"]):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("m,n,k", [(33, 272, 256), (300, 528, 384), (4096, 1024, 1024)])
def test_debug_build_w8a8_no_violation_and_identical(libs, m, n, k):
    rel, dbg = libs
    _violations(dbg)
    g = torch.Generator(device=DEV).manual_seed(m + n + k)
    qa = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=DEV, generator=g)
    qw = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=DEV, generator=g)
    sa = torch.rand(m, device=DEV, generator=g) * 1e-2
    sw = torch.rand(n, device=DEV, generator=g) * 1e-2
    bias = torch.randn(n, device=DEV, generator=g).to(torch.bfloat16)
    outs = {}
    for name, lib in (("rel", rel), ("dbg", dbg)):
        res = []
        for tile in (0, 1):
            lib.gwa_w8a8_gemm_force_tile(tile)
            out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
            _ok(lib.gwa_w8a8_gemm(qa.data_ptr(), qw.data_ptr(), sa.data_ptr(), m, sw.data_ptr(), bias.data_ptr(), 0,
                                  out.data_ptr(), 0, m, n, k, torch.cuda.current_stream().cuda_stream), lib)
            res.append(out)
        lib.gwa_w8a8_gemm_force_tile(-1)
        torch.cuda.synchronize()
        outs[name] = res
    bits, first = _violations(dbg)
    assert bits == 0, f"debug checks failed: sites {bits:#x}, first {first:#x}"
    for a, b in zip(outs["rel"], outs["dbg"]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
