"""gen_worker_amd — MI355X (gfx950) SVDQuant int4-g64 / W8A8 int8 quantized-linear path.

Host side of the C-ABI library ``libgen_worker_amd.so``: the
``cozy_gen_worker::*`` torch ops (``ops``), the quantized layer modules
(``svdq``, ``w8a8``, ``awq``, ``nvfp4``), and offline producers. Importing this package registers
the ops; the native library is loaded on first use and is required (there is
no CPU fallback).
"""

from . import ops  # noqa: F401  (registers cozy_gen_worker::* / cozy_kernels::* ops)
from ._native import NativeError, NativeUnavailable, available as native_available, build_info
from .svdq import (SvdqFusedError, SvdqW4A4Linear, build_svdq_w4a4_linear, fold_to_dense,
                   quantize_linear_w4a4, quantize_weight_int4)
from .nvfp4 import Nvfp4Error, Nvfp4Linear, build_nvfp4_linear, quantize_nvfp4_tensor
from .w8a8 import Int8ScaledLinear, W8a8Error, build_int8_linear, quantize_linear_w8a8, quantize_weight_int8

__all__ = [
    "Int8ScaledLinear", "NativeError", "NativeUnavailable", "Nvfp4Error", "Nvfp4Linear", "SvdqFusedError",
    "SvdqW4A4Linear", "W8a8Error", "build_info", "build_int8_linear", "build_nvfp4_linear",
    "build_svdq_w4a4_linear", "fold_to_dense", "native_available", "quantize_linear_w4a4", "quantize_linear_w8a8",
    "quantize_nvfp4_tensor", "quantize_weight_int4", "quantize_weight_int8",
]
