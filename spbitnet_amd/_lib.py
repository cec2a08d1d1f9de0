"""ctypes binding of the C ABI in include/spbitnet_amd.h.

The library is the in-tree build spbitnet_amd/libspbitnet_amd.so (see
spbitnet_amd/build.py).  There is no fallback: if the library is missing the
import fails with an error naming the build command.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  -- load torch's HIP runtime first so the library binds to it

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libspbitnet_amd.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (restype int unless listed in _RESTYPES)
SIGNATURES = {
    "spb_abi_version": [],
    "spb_last_error_string": [],
    "spb_sparse_ternary_unpack": [_P, _P, _P, _I, _I, _I, _I, _P],
    "spb_sparse_ternary_gemv": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "spb_fused_sparse_bitlinear_f16": [_P, _P, _P, _P, _P, _F, _I, _I, _I, _I, _P],
    "spb_fused_sparse_bitlinear_bf16": [_P, _P, _P, _P, _P, _F, _I, _I, _I, _I, _P],
    "spb_absmax_reduce_f16": [_P, _P, _I, _P],
    "spb_absmax_reduce_bf16": [_P, _P, _I, _P],
    "spb_absmax_quantize_f16": [_P, _P, _P, _I, _P],
    "spb_absmax_quantize_bf16": [_P, _P, _P, _I, _P],
    "spb_dequantize_f16": [_P, _P, _P, _F, _I, _P],
    "spb_dequantize_bf16": [_P, _P, _P, _F, _I, _P],
    "spb_sparse_ternary_gemv_kernel_id": [_P, _P, _I, _I, _I, _I],
    "spb_activation_planes": [_P, _P, _I, _P],
    "spb_sparse_ternary_gemm": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "spb_sparse_ternary_gemm_addsub": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "spb_sparse_ternary_gemm_kernel_id": [_P, _P, _P, _I, _I, _I, _I, _I],
    "spb_absmax_quantize_planes_f16": [_P, _P, _P, _P, _I, _P],
    "spb_absmax_quantize_planes_bf16": [_P, _P, _P, _P, _I, _P],
    "spb_sparse_ternary_gemv_planes": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "spb_fused_sparse_bitlinear_planes_f16": [_P, _P, _P, _P, _P, _F, _I, _I, _I, _I, _P],
    "spb_fused_sparse_bitlinear_planes_bf16": [_P, _P, _P, _P, _P, _F, _I, _I, _I, _I, _P],
}
_RESTYPES = {"spb_last_error_string": ctypes.c_char_p}

_lib = None


class SpbError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python spbitnet_amd/build.py`")
        L = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, _I)
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().spb_last_error_string() or b""
        raise SpbError(f"{what} failed with status {rc}: {msg.decode(errors='replace')}")
