"""Python mirror of the reference's kernel host API for the sparse-ternary
path (include/spbitnet/sparse_ternary_kernels.h:16-48 and
include/spbitnet/inference_kernels.h:19-30 of the reference): same names,
same argument order and meaning, device tensors in place of raw pointers.

Each call checks on the host that every tensor is on the GPU, has the dtype
the kernel expects, is contiguous and is at least as large as the shape
arguments require, then launches through the C ABI on the given stream
(default: torch's current stream).  Failures raise SpbError; rows == 0 or
cols == 0 is a no-op, as in the reference.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

_HALF_KIND = {torch.float16: "f16", torch.bfloat16: "bf16"}


def _stream_ptr(stream) -> Optional[int]:
    if stream is None:
        stream = torch.cuda.current_stream()
    if isinstance(stream, int):
        return stream or None
    return stream.cuda_stream or None


def _dev(t: torch.Tensor, name: str, dtype, min_numel: int) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < min_numel:
        raise ValueError(f"{name} holds {t.numel()} elements, needs at least {min_numel}")
    return t.data_ptr()


def _weights(meta, values, rows, cols, meta_row_stride, values_row_stride):
    if rows < 0 or cols < 0:
        raise ValueError(f"negative shape ({rows}, {cols})")
    if cols % 4:
        raise ValueError(f"cols={cols} is not a multiple of 4")
    if meta_row_stride < (cols // 4 + 7) // 8 or values_row_stride < (cols // 4 + 15) // 16:
        raise ValueError("row strides are smaller than the format requires")
    need_m = rows * meta_row_stride if rows and cols else 0
    need_v = rows * values_row_stride if rows and cols else 0
    pm = _dev(meta, "meta", (torch.int32, torch.uint32), need_m)
    pv = _dev(values, "values", (torch.int32, torch.uint32), need_v)
    return pm, pv


def sparse_ternary_unpack_gpu(meta, values, out, rows, cols, meta_row_stride,
                              values_row_stride, stream=None):
    """reference src/kernels/sparse_ternary.cu:240-254"""
    pm, pv = _weights(meta, values, rows, cols, meta_row_stride, values_row_stride)
    po = _dev(out, "out", torch.int8, rows * cols)
    _lib.check(_lib.load().spb_sparse_ternary_unpack(pm, pv, po, rows, cols, meta_row_stride,
                                                     values_row_stride, _stream_ptr(stream)),
               "sparse_ternary_unpack_gpu")


def sparse_ternary_gemv_gpu(meta, values, x, y, rows, cols, meta_row_stride,
                            values_row_stride, stream=None, resident=False):
    """reference src/kernels/sparse_ternary.cu:256-272 (int8 x -> int32 y).
    resident=True loads the weights on the default cache policy
    (spb_sparse_ternary_gemv_resident: matrices that stay in the Infinity
    Cache between calls) instead of the streaming one."""
    pm, pv = _weights(meta, values, rows, cols, meta_row_stride, values_row_stride)
    empty = rows == 0 or cols == 0
    px = _dev(x, "x", torch.int8, 0 if empty else cols)
    py = _dev(y, "y", torch.int32, 0 if empty else rows)
    L = _lib.load()
    fn = L.spb_sparse_ternary_gemv_resident if resident else L.spb_sparse_ternary_gemv
    _lib.check(fn(pm, pv, px, py, rows, cols, meta_row_stride, values_row_stride,
                  _stream_ptr(stream)), "sparse_ternary_gemv_gpu")


def fused_sparse_bitlinear_gpu(meta, values, x, output, d_absmax, gamma, rows, cols,
                               meta_row_stride, values_row_stride, stream=None):
    """reference src/kernels/sparse_ternary.cu:274-291; x/output fp16 or bf16."""
    pm, pv = _weights(meta, values, rows, cols, meta_row_stride, values_row_stride)
    if x.dtype not in _HALF_KIND:
        raise TypeError("x must be float16 or bfloat16")
    kind = _HALF_KIND[x.dtype]
    empty = rows == 0 or cols == 0
    px = _dev(x, "x", x.dtype, 0 if empty else cols)
    po = _dev(output, "output", x.dtype, 0 if empty else rows)
    pa = _dev(d_absmax, "d_absmax", torch.float32, 1)
    fn = getattr(_lib.load(), f"spb_fused_sparse_bitlinear_{kind}")
    _lib.check(fn(pm, pv, px, po, pa, float(gamma), rows, cols, meta_row_stride,
                  values_row_stride, _stream_ptr(stream)), "fused_sparse_bitlinear_gpu")


def absmax_reduce_gpu(input, d_absmax, size, stream=None):
    """reference src/kernels/inference_kernels.cu:549-553"""
    if input.dtype not in _HALF_KIND:
        raise TypeError("input must be float16 or bfloat16")
    pi = _dev(input, "input", input.dtype, size)
    pa = _dev(d_absmax, "d_absmax", torch.float32, 1)
    fn = getattr(_lib.load(), f"spb_absmax_reduce_{_HALF_KIND[input.dtype]}")
    _lib.check(fn(pi, pa, size, _stream_ptr(stream)), "absmax_reduce_gpu")


def absmax_quantize_gpu(input, output, d_absmax, size, stream=None):
    """reference src/kernels/inference_kernels.cu:543-547"""
    if input.dtype not in _HALF_KIND:
        raise TypeError("input must be float16 or bfloat16")
    pi = _dev(input, "input", input.dtype, size)
    po = _dev(output, "output", torch.int8, size)
    pa = _dev(d_absmax, "d_absmax", torch.float32, 1)
    fn = getattr(_lib.load(), f"spb_absmax_quantize_{_HALF_KIND[input.dtype]}")
    _lib.check(fn(pi, po, pa, size, _stream_ptr(stream)), "absmax_quantize_gpu")


def dequantize_gpu(input, output, d_absmax, gamma, size, stream=None):
    """reference src/kernels/inference_kernels.cu:555-561; output fp16 or bf16."""
    if output.dtype not in _HALF_KIND:
        raise TypeError("output must be float16 or bfloat16")
    pi = _dev(input, "input", torch.int32, size)
    po = _dev(output, "output", output.dtype, size)
    pa = _dev(d_absmax, "d_absmax", torch.float32, 1)
    fn = getattr(_lib.load(), f"spb_dequantize_{_HALF_KIND[output.dtype]}")
    _lib.check(fn(pi, po, pa, float(gamma), size, _stream_ptr(stream)), "dequantize_gpu")


# ---- batched GEMM (replaces the reference's cuSPARSELt path) ------------------

def sparse_ternary_gemm_gpu(meta, values, X, Y, rows, cols, n, meta_row_stride,
                            values_row_stride, stream=None, kernel="auto"):
    """Y[t][r] = sum_c W[r][c] X[t][c] (int32), X int8 [n][cols], Y int32 [n][rows].

    Replaces CuSparseLtGemm::execute (reference src/cusparselt_backend.cu:186-207);
    kernel="auto" uses the matrix-core kernel where the shape allows,
    kernel="addsub" the bit-plane GEMV kernel over tokens (the comparator)."""
    pm, pv = _weights(meta, values, rows, cols, meta_row_stride, values_row_stride)
    if n < 0:
        raise ValueError("negative batch")
    empty = rows == 0 or cols == 0 or n == 0
    px = _dev(X, "X", torch.int8, 0 if empty else n * cols)
    py = _dev(Y, "Y", torch.int32, 0 if empty else n * rows)
    L = _lib.load()
    fn = L.spb_sparse_ternary_gemm if kernel == "auto" else L.spb_sparse_ternary_gemm_addsub
    _lib.check(fn(pm, pv, px, py, rows, cols, n, meta_row_stride, values_row_stride,
                  _stream_ptr(stream)), "sparse_ternary_gemm_gpu")


def gemm_kernel_id(meta, values, X, rows, cols, n, meta_row_stride, values_row_stride) -> int:
    """Kernel spb_sparse_ternary_gemm would run for these arguments: 2 the
    staged matrix-core kernel, 1 the direct matrix-core kernel, 0 the general
    kernel."""
    return _lib.load().spb_sparse_ternary_gemm_kernel_id(
        meta.data_ptr(), values.data_ptr(), X.data_ptr(), rows, cols, n, meta_row_stride,
        values_row_stride)


# ---- 2:4 structured-sparse int8 GEMM (the cuSPARSELt backend) ---------------

def sparse_i8_compressed_size(m: int, k: int) -> int:
    """Bytes of the compressed operand of an m x k int8 matrix (the size query
    of cusparseLtSpMMACompressedSize, reference src/cusparselt_backend.cu:140-146)."""
    L = _lib.load()
    n = L.spb_sparse_i8_compressed_size(m, k)
    if n < 0:
        _lib.check(1, "sparse_i8_compressed_size")
    return int(n)


def sparse_i8_prune_check(d_weights, m: int, k: int, stream=None) -> int:
    """Groups of the int8 [m][k] matrix with more than two non-zeros
    (0 = already 2:4), cusparseLtSpMMAPruneCheck as prepare uses it
    (reference src/cusparselt_backend.cu:123-136)."""
    pa = _dev(d_weights, "d_weights", torch.int8, m * k)
    res = torch.empty(1, dtype=torch.int32, device=d_weights.device)
    _lib.check(_lib.load().spb_sparse_i8_prune_check(pa, m, k, res.data_ptr(),
                                                       _stream_ptr(stream)),
               "sparse_i8_prune_check")
    return int(res.item())


class CuSparseLtGemm:
    """CuSparseLtGemm (reference include/spbitnet/cusparselt_backend.h:28-77,
    src/cusparselt_backend.cu:38-219): D[m,n] = A_pruned[m,k] * B[k,n] with
    int32 accumulation on the int8 sparse matrix cores.

    prepare(d_weights) prunes a device int8 [m][k] row-major matrix (any int8
    values, k a multiple of 4) to 2:4 along k -- the two largest |a| of each
    group of four, on equal magnitudes the higher index; groups with at most
    two non-zeros are kept whole -- and compresses it into a device buffer
    this object owns.  execute(d_B, d_D) takes B int8 [k x n] column-major
    (a [n][k] tensor) and writes D int32 [m x n] column-major (a [n][m]
    tensor).  Any n >= 1 (the reference needs n >= 16)."""

    def __init__(self, m: int, k: int, n: int, device="cuda"):
        if n < 1:
            raise ValueError("n must be >= 1")
        self._m, self._k, self._n = m, k, n
        size = sparse_i8_compressed_size(m, k)
        self._comp = torch.empty(max(size, 16), dtype=torch.uint8, device=device)
        self._prepared = False

    def m(self) -> int:
        return self._m

    def k(self) -> int:
        return self._k

    def n(self) -> int:
        return self._n

    def prepare(self, d_weights, stream=None) -> None:
        """Prune to 2:4 and compress (src/cusparselt_backend.cu:107-166)."""
        pa = _dev(d_weights, "d_weights", torch.int8, self._m * self._k)
        _lib.check(_lib.load().spb_sparse_i8_prune_compress(
            pa, None, self._comp.data_ptr(), self._m, self._k, _stream_ptr(stream)),
            "CuSparseLtGemm.prepare")
        self._prepared = True

    def execute(self, d_B, d_D, stream=None) -> None:
        """D = A_pruned * B (src/cusparselt_backend.cu:173-207)."""
        if not self._prepared:
            raise RuntimeError("CuSparseLtGemm.execute() called before prepare()")
        pb = _dev(d_B, "d_B", torch.int8, self._n * self._k)
        pd = _dev(d_D, "d_D", torch.int32, self._n * self._m)
        _lib.check(_lib.load().spb_sparse_i8_gemm(self._comp.data_ptr(), pb, pd, self._m,
                                                    self._k, self._n, _stream_ptr(stream)),
                   "CuSparseLtGemm.execute")

    def get_pruned_weights(self, d_out, stream=None) -> None:
        """The pruned dense int8 [m][k] matrix (src/cusparselt_backend.cu:209-217)."""
        if not self._prepared:
            raise RuntimeError("CuSparseLtGemm.get_pruned_weights(): not prepared")
        po = _dev(d_out, "d_out", torch.int8, self._m * self._k)
        _lib.check(_lib.load().spb_sparse_i8_decompress(self._comp.data_ptr(), po, self._m,
                                                          self._k, _stream_ptr(stream)),
                   "CuSparseLtGemm.get_pruned_weights")

    def kernel_id(self, d_B) -> int:
        """1 when execute runs the matrix-core kernel for d_B, 0 the general one."""
        return _lib.load().spb_sparse_i8_gemm_kernel_id(self._comp.data_ptr(), d_B.data_ptr(),
                                                        self._m, self._k, self._n)


# ---- bit-plane activation layout (no reference counterpart) -----------------

def planes_words(cols: int) -> int:
    """uint32 words of the plane layout of a `cols`-column activation."""
    return 8 * ((cols + 31) // 32)


def activation_planes_gpu(x, planes, cols, stream=None):
    """int8 x[cols] -> bit-plane layout (word [w*8+b] = plane b of columns 32w..32w+31)."""
    px = _dev(x, "x", torch.int8, cols)
    pp = _dev(planes, "planes", (torch.int32, torch.uint32), planes_words(cols))
    _lib.check(_lib.load().spb_activation_planes(px, pp, cols, _stream_ptr(stream)),
               "activation_planes_gpu")


def absmax_quantize_planes_gpu(input, planes, d_absmax, size, output=None, stream=None):
    """absmax + int8 quantisation emitting the plane layout (and the int8 vector if given)."""
    if input.dtype not in _HALF_KIND:
        raise TypeError("input must be float16 or bfloat16")
    pi = _dev(input, "input", input.dtype, size)
    pp = _dev(planes, "planes", (torch.int32, torch.uint32), planes_words(size))
    pa = _dev(d_absmax, "d_absmax", torch.float32, 1)
    po = _dev(output, "output", torch.int8, size) if output is not None else None
    fn = getattr(_lib.load(), f"spb_absmax_quantize_planes_{_HALF_KIND[input.dtype]}")
    _lib.check(fn(pi, pp, po, pa, size, _stream_ptr(stream)), "absmax_quantize_planes_gpu")


def sparse_ternary_gemv_planes_gpu(meta, values, planes, y, rows, cols, meta_row_stride,
                                   values_row_stride, stream=None):
    """sparse_ternary_gemv_gpu with plane-layout activations."""
    pm, pv = _weights(meta, values, rows, cols, meta_row_stride, values_row_stride)
    empty = rows == 0 or cols == 0
    pp = _dev(planes, "planes", (torch.int32, torch.uint32), 0 if empty else planes_words(cols))
    py = _dev(y, "y", torch.int32, 0 if empty else rows)
    _lib.check(_lib.load().spb_sparse_ternary_gemv_planes(pm, pv, pp, py, rows, cols,
                                                          meta_row_stride, values_row_stride,
                                                          _stream_ptr(stream)),
               "sparse_ternary_gemv_planes_gpu")


def fused_sparse_bitlinear_planes_gpu(meta, values, planes, output, d_absmax, gamma, rows, cols,
                                      meta_row_stride, values_row_stride, stream=None):
    """GEMV on plane activations + the reference's dequant epilogue; output fp16 or bf16."""
    pm, pv = _weights(meta, values, rows, cols, meta_row_stride, values_row_stride)
    if output.dtype not in _HALF_KIND:
        raise TypeError("output must be float16 or bfloat16")
    empty = rows == 0 or cols == 0
    pp = _dev(planes, "planes", (torch.int32, torch.uint32), 0 if empty else planes_words(cols))
    po = _dev(output, "output", output.dtype, 0 if empty else rows)
    pa = _dev(d_absmax, "d_absmax", torch.float32, 1)
    fn = getattr(_lib.load(), f"spb_fused_sparse_bitlinear_planes_{_HALF_KIND[output.dtype]}")
    _lib.check(fn(pm, pv, pp, po, pa, float(gamma), rows, cols, meta_row_stride,
                  values_row_stride, _stream_ptr(stream)), "fused_sparse_bitlinear_planes_gpu")


def gemv_kernel_id(meta, values, rows, cols, meta_row_stride, values_row_stride) -> int:
    """1 if the bit-plane GEMV kernel would run for these arguments, else 0."""
    return _lib.load().spb_sparse_ternary_gemv_kernel_id(
        meta.data_ptr(), values.data_ptr(), rows, cols, meta_row_stride, values_row_stride)


def bitlinear_workspace_size(cols: int) -> int:
    """Bytes of the workspace bitlinear_gpu needs for `cols` input columns."""
    return int(_lib.load().spb_bitlinear_workspace_size(int(cols)))


def bitlinear_gpu(meta, values, x, output, gamma, rows, cols, meta_row_stride,
                  values_row_stride, workspace, stream=None):
    """InferenceEngine::bitlinear (reference src/inference.cu:106-117) as one
    call: absmax, quantisation, sparse GEMV and dequantisation, with the
    absmax scratch (and the activation planes) in `workspace`, a uint8 GPU
    tensor of at least bitlinear_workspace_size(cols) bytes."""
    pm, pv = _weights(meta, values, rows, cols, meta_row_stride, values_row_stride)
    empty = rows == 0 or cols == 0
    kind = _HALF_KIND.get(x.dtype)
    if kind is None:
        raise TypeError(f"x has dtype {x.dtype}, expected float16 or bfloat16")
    px = _dev(x, "x", x.dtype, 0 if empty else cols)
    po = _dev(output, "output", x.dtype, 0 if empty else rows)
    need = 0 if empty else bitlinear_workspace_size(cols)
    pw = _dev(workspace, "workspace", torch.uint8, need)
    fn = getattr(_lib.load(), f"spb_bitlinear_{kind}")
    _lib.check(fn(pm, pv, px, po, float(gamma), rows, cols, meta_row_stride, values_row_stride,
                  pw, workspace.numel(), _stream_ptr(stream)), "bitlinear_gpu")
