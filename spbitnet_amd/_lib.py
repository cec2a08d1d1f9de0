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
    "spb_sparse_ternary_gemv_resident": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
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
    "spb_bitlinear_workspace_size": [_I],
    "spb_bitlinear_f16": [_P, _P, _P, _P, _F, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "spb_bitlinear_bf16": [_P, _P, _P, _P, _F, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "spb_bitlinear_f16_noalloc": [_P, _P, _P, _P, _F, _I, _I, _I, _I, _P],
    "spb_bitlinear_bf16_noalloc": [_P, _P, _P, _P, _F, _I, _I, _I, _I, _P],
    # per-op inference kernels
    "spb_rms_norm_f16": [_P, _P, _P, _I, _F, _P],
    "spb_rms_norm_bf16": [_P, _P, _P, _I, _F, _P],
    "spb_rms_norm_f32in_f16": [_P, _P, _P, _I, _F, _P],
    "spb_rms_norm_f32in_bf16": [_P, _P, _P, _I, _F, _P],
    "spb_rope_f16": [_P, _I, _I, _I, _F, _P],
    "spb_rope_bf16": [_P, _I, _I, _I, _F, _P],
    "spb_scatter_kv": [_P, _P, _I, _I, _I, _I, _P],
    "spb_attention_scores_f16": [_P, _P, _P, _I, _I, _I, _I, _I, _F, _P],
    "spb_attention_scores_bf16": [_P, _P, _P, _I, _I, _I, _I, _I, _F, _P],
    "spb_softmax": [_P, _I, _I, _I, _P],
    "spb_attention_output_f16": [_P, _P, _P, _I, _I, _I, _I, _I, _P],
    "spb_attention_output_bf16": [_P, _P, _P, _I, _I, _I, _I, _I, _P],
    "spb_relu2_mul_f16": [_P, _P, _P, _I, _P],
    "spb_relu2_mul_bf16": [_P, _P, _P, _I, _P],
    "spb_relu2_mul_f32_f16": [_P, _P, _P, _I, _P],
    "spb_relu2_mul_f32_bf16": [_P, _P, _P, _I, _P],
    "spb_float_to_f16": [_P, _P, _I, _P],
    "spb_float_to_bf16": [_P, _P, _I, _P],
    "spb_residual_add_f16": [_P, _P, _P, _I, _P],
    "spb_residual_add_bf16": [_P, _P, _P, _I, _P],
    "spb_gemv_f16": [_P, _P, _P, _I, _I, _P],
    "spb_gemv_bf16": [_P, _P, _P, _I, _I, _P],
    "spb_argmax_f32": [_P, _I, _P, _P],
    # decode engine (structs passed by pointer)
    "spb_engine_create": [_P, _P, _P, _P, _P, _I, _P],
    "spb_engine_destroy": [_P],
    "spb_engine_set_stream": [_P, _P],
    "spb_engine_reset": [_P],
    "spb_engine_forward": [_P, _I, _P],
    "spb_engine_seq_len": [_P],
    "spb_engine_generate": [_P, _P, _I, _I, _I, _P, _P],
    "spb_engine_decode_steps": [_P, _I],
    "spb_engine_set_prefill_batch": [_P, _I],
    "spb_engine_buffers": [_P, _P, _P],
    "spb_batch_engine_create": [_P, _P, _P, _P, _P, _I, _I, _P],
    "spb_batch_engine_destroy": [_P],
    "spb_batch_engine_set_stream": [_P, _P],
    "spb_batch_engine_generate": [_P, _P, _P, _I, _I, _I, _P, _P],
    "spb_batch_engine_decode_steps": [_P, _I],
    "spb_batch_engine_buffers": [_P, _P, _P],
    "spb_model_load": [ctypes.c_char_p, _P],
    "spb_model_destroy": [_P],
    "spb_model_info": [_P, _P, _P, _P, _P, _P, _P],
    "spb_generate_sparse_ternary": [ctypes.c_uint64, _I, _I, _P, _P, _I, _I, _P, _P, _P],
    "spb_generate_normal_bf16": [ctypes.c_uint64, ctypes.c_long, _F, _P, _P],
    # 2:4 structured-sparse int8 GEMM (the cuSPARSELt backend)
    "spb_sparse_i8_compressed_size": [_I, _I],
    "spb_sparse_i8_prune_compress": [_P, _P, _P, _I, _I, _P],
    "spb_sparse_i8_prune_check": [_P, _I, _I, _P, _P],
    "spb_sparse_i8_decompress": [_P, _P, _I, _I, _P],
    "spb_sparse_i8_gemm": [_P, _P, _P, _I, _I, _I, _P],
    "spb_sparse_i8_gemm_kernel_id": [_P, _P, _I, _I, _I],
}
_RESTYPES = {"spb_last_error_string": ctypes.c_char_p,
             "spb_bitlinear_workspace_size": ctypes.c_size_t,
             "spb_sparse_i8_compressed_size": ctypes.c_long}


class SparseLinearC(ctypes.Structure):
    """spb_sparse_linear (include/spbitnet_amd.h)."""
    _fields_ = [("meta", _P), ("values", _P), ("gamma", _F), ("rows", _I), ("cols", _I),
                ("meta_stride", _I), ("values_stride", _I)]


class TransformerLayerC(ctypes.Structure):
    """spb_transformer_layer (include/spbitnet_amd.h)."""
    _fields_ = [(n, SparseLinearC) for n in
                ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")] + \
               [("input_layernorm", _P), ("post_attention_layernorm", _P),
                ("attn_sub_norm", _P), ("ffn_sub_norm", _P)]


class ModelConfigC(ctypes.Structure):
    """spb_model_config (include/spbitnet_amd.h)."""
    _fields_ = [(n, _I) for n in ("hidden_size", "num_hidden_layers", "num_attention_heads",
                                  "num_key_value_heads", "intermediate_size", "vocab_size",
                                  "max_position_embeddings", "head_dim")] + \
               [("rms_norm_eps", _F), ("rope_theta", _F), ("bos_token_id", _I),
                ("eos_token_id", _I)]

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


_hip = None


def memcpy_d2d(dst: int, src: int, nbytes: int, stream) -> None:
    """Device-to-device copy on `stream` through the HIP runtime torch loaded."""
    global _hip
    if _hip is None:
        path = os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so")
        _hip = ctypes.CDLL(path if os.path.exists(path) else "libamdhip64.so")
        _hip.hipMemcpyAsync.argtypes = [_P, _P, ctypes.c_size_t, _I, _P]
        _hip.hipMemcpyAsync.restype = _I
    rc = _hip.hipMemcpyAsync(dst, src, nbytes, 3, stream)  # 3 = hipMemcpyDeviceToDevice
    if rc != 0:
        raise SpbError(f"hipMemcpyAsync failed with status {rc}")
