"""ctypes binding of the C-ABI library ``libgen_worker_amd.so``.

The library is located next to this file, or at ``$GEN_WORKER_AMD_LIB``.
There is no fallback: a missing or unloadable library raises
:class:`NativeUnavailable`, and every failed call raises
:class:`NativeError` with the library's own message (the equivalents of the
``TORCH_CHECK`` / launch-check failures of ``csrc/cozy_kernels/probe.cu:15-25``
in the reference).
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path
from typing import Optional

LIB_ENV = "GEN_WORKER_AMD_LIB"
LIB_NAME = "libgen_worker_amd.so"

DT_BF16, DT_F16, DT_F32 = 0, 1, 2
EPI_GELU_TANH = 1
NVFP4_SCALES_FLAT, NVFP4_SCALES_BLOCKED = 0, 1
EPI_LA_F32 = 2
QFMT_INT4, QFMT_FP6 = 0, 1
FP6_REC = 104   # bytes per fp6 operand record (GWA_FP6_REC)


class NativeUnavailable(RuntimeError):
    """The HIP extension library could not be found or loaded."""


class NativeError(RuntimeError):
    """A C-ABI call returned an error code."""


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float

# name -> argtypes (all return int status unless listed in _RESTYPES)
_SIGNATURES: dict[str, tuple] = {
    "gwa_version": (),
    "gwa_build_info": (),
    "gwa_last_error": (),
    "gwa_probe_add_one": (_vp, _vp, _i64, _vp),
    "gwa_svdq_quant_int4": (_vp, _i64, _vp, _vp, _vp, _i64, _int, _vp, _vp, _vp, _i64, _i64, _vp),
    "gwa_svdq_prep_proj_down": (_vp, _vp, _i64, _i64, _vp),
    "gwa_svdq_gemm_w4a4": (_vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _int, _int,
                           _i64, _i64, _i64, _vp),
    "gwa_svdq_group_psums": (_vp, _vp, _vp, _i64, _i64, _i64, _vp),
    "gwa_svdq_pack_weight_fp6": (_vp, _vp, _vp, _i64, _i64, _vp),
    "gwa_svdq_gemm_w4a4_fp6": (_vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _int, _int,
                               _i64, _i64, _i64, _vp),
    "gwa_svdq_group_psums_fp6": (_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp),
    "gwa_svdq_w4a4_linear_fp6": (_vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _int, _int,
                                 _i64, _i64, _i64, _vp, _i64, _vp),
    "gwa_svdq_w4a4_linear_fp6_workspace": (_i64, _i64, _i64),
    "gwa_svdq_w4a4_linear_fp6_noalloc": (_vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp,
                                         _int, _int, _i64, _i64, _i64, _vp),
    "gwa_svdq_w4a4_linear_fp6_noalloc_scratch_bytes": (),
    "gwa_svdq_w4a4_linear_gemv": (_vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _int, _int,
                                  _i64, _i64, _i64, _vp, _i64, _vp),
    "gwa_svdq_w4a4_gemv_max_m": (_i64, _i64),
    "gwa_svdq_w4a4_linear_gemv_workspace": (_i64, _i64, _i64),
    "gwa_svdq_gemm_w4a4_fp6_next": (_vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _int,
                                    _vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp),
    "gwa_svdq_quant_fp6": (_vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _vp),
    "gwa_svdq_prep_proj_down_fp6": (_vp, _vp, _i64, _i64, _vp),
    "gwa_svdq_quant_fp6_partials": (_i64, _i64, _i64),
    "gwa_svdq_quant_fp6_la": (_vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _vp),
    "gwa_svdq_quant_fp6_la_workspace": (_i64, _i64, _i64),
    "gwa_debug_violations": (ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64), _int),
    "gwa_svdq_gemm_w4a4_fp6_next_partials": (_i64, _i64),
    "gwa_svdq_gemm_w4a4_fp6_tile": (_i64, _i64),
    "gwa_svdq_gemm_w4a4_fp6_force_tile": (_int,),
    "gwa_svdq_la_reduce": (_vp, _i64, _i64, _i64, _vp, _vp),
    "gwa_svdq_epilogue_lora": (_vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _vp),
    "gwa_w8a8_quant_int8": (_vp, _i64, _vp, _vp, _i64, _i64, _vp),
    "gwa_w8a8_quant": (_vp, _i64, _vp, _vp, _vp, _int, _vp, _i64, _i64, _vp),
    "gwa_w8a8_gemm": (_vp, _vp, _vp, _i64, _vp, _vp, _int, _vp, _int, _i64, _i64, _i64, _vp),
    "gwa_w8a8_gemm_tile": (_i64, _i64, _i64),
    "gwa_w8a8_gemm_force_tile": (_int,),
    "gwa_awq_w4a16_mm": (_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp),
    "gwa_dit_qk_norm_rope": (_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64,
                             _i64, _i64, _flt, _vp),
    "gwa_dit_adaln_modulate": (_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _flt, _vp),
    "gwa_dit_gate_residual": (_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp),
    "gwa_dit_attention": (_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _flt, _vp),
    "gwa_awq_w4a16_dequant": (_vp, _vp, _vp, _vp, _i64, _i64, _vp),
    "gwa_transpose_2d": (_vp, _vp, _i64, _i64, _i64, _vp),
    "gwa_nvfp4_blocked_scale_numel": (_i64, _i64),
    "gwa_nvfp4_quant_act": (_vp, _i64, _vp, _vp, _vp, _int, _vp, _i64, _i64, _vp),
    "gwa_nvfp4_quant_act_dyn": (_vp, _i64, _vp, _vp, _vp, _vp, _int, _vp, _i64, _i64, _vp),
    "gwa_nvfp4_dequant": (_vp, _vp, _int, _vp, _i64, _i64, _vp),
    "gwa_nvfp4_scale_bias": (_vp, _vp, _vp, _vp, _i64, _i64, _vp),
}
_RESTYPES = {"gwa_build_info": ctypes.c_char_p, "gwa_last_error": ctypes.c_char_p,
             "gwa_svdq_quant_fp6_partials": ctypes.c_int64, "gwa_svdq_gemm_w4a4_fp6_next_partials": ctypes.c_int64,
             "gwa_nvfp4_blocked_scale_numel": ctypes.c_int64, "gwa_svdq_w4a4_linear_fp6_workspace": ctypes.c_int64,
             "gwa_svdq_w4a4_linear_fp6_noalloc_scratch_bytes": ctypes.c_int64,
             "gwa_svdq_quant_fp6_la_workspace": ctypes.c_int64,
             "gwa_svdq_w4a4_linear_gemv_workspace": ctypes.c_int64}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def library_path() -> Path:
    override = os.environ.get(LIB_ENV, "").strip()
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / LIB_NAME


DEBUG_LIB_NAME = "libgen_worker_amd_debug.so"


def debug_library_path() -> Path:
    """The GWA_DEBUG build of the same sources (device-side bounds checks; ``gwa_debug_violations`` reads
    them), built beside the library by ``build()``."""
    return Path(__file__).resolve().parent / DEBUG_LIB_NAME


def load_debug() -> ctypes.CDLL:
    """Load the debug build as a second, independent library (its own kernels and state); raises
    :class:`NativeUnavailable` when it is not built."""
    path = debug_library_path()
    if not path.exists():
        raise NativeUnavailable(f"{path} does not exist: `python -m gen_worker_amd.build` builds it")
    import torch  # noqa: F401  (the HIP runtime torch loaded)
    lib = ctypes.CDLL(str(path))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            raise NativeUnavailable(f"{path} does not export {name}")
        fn.argtypes = list(argtypes)
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    return lib


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises :class:`NativeUnavailable`."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise NativeUnavailable(
                f"{path} does not exist: build it with `python -m gen_worker_amd.build` "
                f"(or __graft_entry__.build()); there is no CPU fallback")
        try:
            # torch's HIP runtime (same soname) must be the one the library binds to
            import torch  # noqa: F401
            lib = ctypes.CDLL(str(path))
        except OSError as exc:
            raise NativeUnavailable(f"{path} failed to load: {exc}") from exc
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise NativeUnavailable(f"{path} does not export {name}")
            fn.argtypes = list(argtypes)
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except NativeUnavailable:
        return False


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point; raise NativeError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.gwa_last_error().decode(errors="replace")
        raise NativeError(f"{name} failed (code {rc}): {msg}")


def build_info() -> str:
    return load().gwa_build_info().decode()


def ptr(t) -> Optional[int]:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    import torch

    return torch.cuda.current_stream(t.device).cuda_stream
