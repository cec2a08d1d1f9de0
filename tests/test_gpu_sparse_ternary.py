"""GPU parity of the sparse-ternary kernels against the CPU oracle.

Mirrors the reference's tests/test_sparse_ternary.cu (UnpackMatchesCPU,
GemvCorrectness, GemvLargeDimension) on the golden vectors regenerated from
those tests, then covers every shape of BASELINE configs 0/1/4, odd and
empty shapes, both GEMV kernels, padded strides, accumulator extremes and the
fused BitLinear / quantiser / dequantiser entry points.  Integer outputs
must match bit for bit; fp16/bf16 outputs are compared as bit patterns too
(the float32 operation order is the reference's, so they are exact).
"""
import hashlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spbitnet_amd import kernels as K
from spbitnet_amd import weights as W

pytestmark = pytest.mark.gpu

CONFIG_SHAPES = [(2560, 2560), (6912, 2560), (2560, 6912), (640, 2560), (2048, 2048),
                 (5632, 2048), (2048, 5632), (8192, 2560)]


def dev_u32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to(device)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def run_gemv(meta, values, x, rows, cols, device, ms=None, vs=None):
    ms = ms or meta.shape[1]
    vs = vs or values.shape[1]
    d_y = torch.full((rows,), -7, dtype=torch.int32, device=device)
    K.sparse_ternary_gemv_gpu(dev_u32(meta, device), dev_u32(values, device), dev(x, device), d_y,
                              rows, cols, ms, vs)
    torch.cuda.synchronize()
    return d_y.cpu().numpy()


def quantized_activation(n, seed, relu2=False):
    if relu2:  # down-projection input: relu(g)^2 * u
        g = W.normal_f32(seed, n)
        u = W.normal_f32(seed + 1, n)
        a = (np.maximum(g, 0) ** 2 * u).astype(np.float32)
    else:
        a = W.normal_f32(seed, n)
    q, _ = W.quantize_absmax_host(a)
    return q


# ---- the reference's own GPU tests ------------------------------------------

def test_unpack_matches_cpu(gpu, golden):
    meta, values = golden["unpack8x64_meta"], golden["unpack8x64_values"]
    out = torch.zeros(8 * 64, dtype=torch.int8, device=gpu)
    K.sparse_ternary_unpack_gpu(dev_u32(meta, gpu), dev_u32(values, gpu), out, 8, 64,
                                meta.shape[1], values.shape[1])
    torch.cuda.synchronize()
    assert (out.cpu().numpy().reshape(8, 64) == golden["unpack8x64_dense"]).all()


def test_gemv_correctness_64x256(gpu, golden):
    y = run_gemv(golden["gemv64x256_meta"], golden["gemv64x256_values"], golden["gemv64x256_x"],
                 64, 256, gpu)
    assert (y == golden["gemv64x256_y"]).all()


def test_gemv_large_dimension_2048(gpu, golden):
    if not O.ref_available():
        pytest.skip("oracle/_ref (reference input generator) not built")
    w, m, x = O.ref_make_test_case(77, 2048, 2048, True)
    meta, values = W.pack(w, m.astype(bool))
    h = hashlib.sha256(meta.tobytes() + values.tobytes()).digest()
    assert h == golden["gemv2048_meta_values_sha256"].tobytes()
    y = run_gemv(meta, values, x, 2048, 2048, gpu)
    assert (y == golden["gemv2048_y"]).all()


# ---- config shapes ------------------------------------------------------------

@pytest.mark.parametrize("rows,cols", CONFIG_SHAPES)
def test_gemv_config_shapes(gpu, rows, cols):
    L = W.random_layer(rows, cols, W.seed_for("cfg", rows, cols))
    x = quantized_activation(cols, W.seed_for("x", rows, cols), relu2=(cols > rows))
    assert K.gemv_kernel_id(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), rows, cols,
                            L.meta_stride, L.values_stride) == 1
    y = run_gemv(L.meta, L.values, x, rows, cols, gpu)
    assert (y == O.gemv(L.meta, L.values, x, rows, cols)).all()


@pytest.mark.parametrize("rows,cols", [(6912, 2560), (2560, 6912), (333, 384), (9, 36)])
def test_gemv_resident_policy(gpu, rows, cols):
    """spb_sparse_ternary_gemv_resident (default cache policy for the weight
    loads) gives the drop-in GEMV's exact products, on both kernels."""
    L = W.random_layer(rows, cols, W.seed_for("resident", rows, cols))
    x = np.random.default_rng(rows + cols).integers(-128, 128, cols).astype(np.int8)
    d_y = torch.full((rows,), -7, dtype=torch.int32, device=gpu)
    K.sparse_ternary_gemv_gpu(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), dev(x, gpu), d_y,
                              rows, cols, L.meta_stride, L.values_stride, resident=True)
    torch.cuda.synchronize()
    assert (d_y.cpu().numpy() == O.gemv(L.meta, L.values, x, rows, cols)).all()


@pytest.mark.parametrize("rows,cols", [(1, 128), (7, 256), (333, 384), (1025, 128), (3, 4),
                                       (5, 8), (9, 36), (64, 100), (130, 132), (31, 2564),
                                       (97, 32768), (1501, 16384), (777, 4992)])
def test_gemv_odd_shapes(gpu, rows, cols):
    L = W.random_layer(rows, cols, W.seed_for("odd", rows, cols))
    x = np.random.default_rng(rows * 7 + cols).integers(-128, 128, cols).astype(np.int8)
    y = run_gemv(L.meta, L.values, x, rows, cols, gpu)
    assert (y == O.gemv(L.meta, L.values, x, rows, cols)).all()


def test_gemv_padded_strides_both_kernels(gpu):
    rows, cols = 77, 512
    L = W.random_layer(rows, cols, 11)
    x = np.random.default_rng(1).integers(-128, 128, cols).astype(np.int8)
    expect = O.gemv(L.meta, L.values, x, rows, cols)
    for pad_m, pad_v in [(4, 2), (1, 0), (0, 1), (3, 3)]:
        meta = np.zeros((rows, L.meta_stride + pad_m), np.uint32)
        values = np.zeros((rows, L.values_stride + pad_v), np.uint32)
        meta[:, :L.meta_stride] = L.meta
        values[:, :L.values_stride] = L.values
        meta[:, L.meta_stride:] = 0xFFFFFFFF      # padding words must never be read
        values[:, L.values_stride:] = 0xFFFFFFFF
        want_kernel = 1 if (pad_m % 4 == 0 and pad_v % 2 == 0) else 0
        assert K.gemv_kernel_id(dev_u32(meta, gpu), dev_u32(values, gpu), rows, cols,
                                meta.shape[1], values.shape[1]) == want_kernel
        y = run_gemv(meta, values, x, rows, cols, gpu)
        assert (y == expect).all(), (pad_m, pad_v)


def test_gemv_accumulator_extremes(gpu):
    rows, cols = 64, 6912
    L = W.random_layer(rows, cols, 12)
    dense = W.unpack(L.meta, L.values, rows, cols)
    xs = [np.full(cols, -128, np.int8), np.full(cols, 127, np.int8),
          np.where(dense[0] < 0, -128, 127).astype(np.int8),
          np.where(dense[1] < 0, 127, -128).astype(np.int8)]
    for x in xs:
        y = run_gemv(L.meta, L.values, x, rows, cols, gpu)
        assert (y == O.gemv(L.meta, L.values, x, rows, cols)).all()


def test_gemv_empty_is_noop(gpu):
    d_y = torch.full((4,), 5, dtype=torch.int32, device=gpu)
    z = torch.zeros(16, dtype=torch.int32, device=gpu)
    K.sparse_ternary_gemv_gpu(z, z, torch.zeros(16, dtype=torch.int8, device=gpu), d_y, 0, 128, 4, 2)
    K.sparse_ternary_gemv_gpu(z, z, torch.zeros(16, dtype=torch.int8, device=gpu), d_y, 4, 0, 0, 0)
    torch.cuda.synchronize()
    assert (d_y.cpu().numpy() == 5).all()


def test_gemv_streamed_copies_property(gpu):
    """Full-size, size-independent check: 40 stacked distinct copies of the
    6912x2560 matrix (one tall GEMV, 132 MB of weights) give each copy's
    single-matrix result, and copy k's rows match the oracle."""
    rows, cols, copies = 6912, 2560, 40
    L = W.random_layer(rows, cols, 21)
    x = quantized_activation(cols, 22)
    y1 = O.gemv(L.meta, L.values, x, rows, cols)
    d_meta = dev_u32(L.meta, gpu).repeat(copies, 1)
    d_values = dev_u32(L.values, gpu).repeat(copies, 1)
    d_y = torch.zeros(rows * copies, dtype=torch.int32, device=gpu)
    K.sparse_ternary_gemv_gpu(d_meta, d_values, dev(x, gpu), d_y, rows * copies, cols,
                              L.meta_stride, L.values_stride)
    torch.cuda.synchronize()
    y = d_y.cpu().numpy().reshape(copies, rows)
    assert (y == y1[None, :]).all()


def test_unpack_config_shape(gpu):
    rows, cols = 640, 2560
    L = W.random_layer(rows, cols, 31)
    out = torch.zeros(rows * cols, dtype=torch.int8, device=gpu)
    K.sparse_ternary_unpack_gpu(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), out, rows, cols,
                                L.meta_stride, L.values_stride)
    torch.cuda.synchronize()
    assert (out.cpu().numpy().reshape(rows, cols) == O.unpack(L.meta, L.values, rows, cols)).all()


def test_gemv_deterministic_on_side_stream(gpu):
    rows, cols = 2560, 6912
    L = W.random_layer(rows, cols, 41)
    x = quantized_activation(cols, 42, relu2=True)
    s = torch.cuda.Stream()
    d_meta, d_values, d_x = dev_u32(L.meta, gpu), dev_u32(L.values, gpu), dev(x, gpu)
    torch.cuda.synchronize()
    outs = []
    for _ in range(3):
        d_y = torch.empty(rows, dtype=torch.int32, device=gpu)
        with torch.cuda.stream(s):
            K.sparse_ternary_gemv_gpu(d_meta, d_values, d_x, d_y, rows, cols, L.meta_stride,
                                      L.values_stride, stream=s)
        s.synchronize()
        outs.append(d_y.cpu().numpy())
    assert all((o == outs[0]).all() for o in outs)
    assert (outs[0] == O.gemv(L.meta, L.values, x, rows, cols)).all()


# ---- quantiser, dequantiser, fused BitLinear -------------------------------

HALF = {"f16": torch.float16, "bf16": torch.bfloat16}


def half_tensor(x_f32, kind, device):
    t = torch.from_numpy(np.asarray(x_f32, np.float32)).to(HALF[kind])
    return t.to(device), t.float().numpy()


def half_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def oracle_half_bits(f32, kind):
    return O.to_f16_bits(f32) if kind == "f16" else O.to_bf16_bits(f32)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("n", [1, 63, 2560, 6912, 100003])
def test_absmax_reduce_and_quantize(gpu, kind, n):
    x, xf = half_tensor(W.normal_f32(W.seed_for("q", n), n) * 3, kind, gpu)
    d_a = torch.zeros(1, dtype=torch.float32, device=gpu)
    K.absmax_reduce_gpu(x, d_a, n)
    q = torch.zeros(n, dtype=torch.int8, device=gpu)
    d_a2 = torch.zeros(1, dtype=torch.float32, device=gpu)
    K.absmax_quantize_gpu(x, q, d_a2, n)
    torch.cuda.synchronize()
    oq, oa = O.quantize(xf)
    assert d_a.item() == oa and d_a2.item() == oa
    assert (q.cpu().numpy() == oq).all()


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_quantize_all_zero(gpu, kind):
    x = torch.zeros(2560, dtype=HALF[kind], device=gpu)
    q = torch.full((2560,), 3, dtype=torch.int8, device=gpu)
    d_a = torch.full((1,), 9.0, dtype=torch.float32, device=gpu)
    K.absmax_quantize_gpu(x, q, d_a, 2560)
    torch.cuda.synchronize()
    assert d_a.item() == 0.0 and (q.cpu().numpy() == 0).all()


def double_rounding_cases(gamma, absmax, kind):
    """Accumulators whose dequantised value rounds differently when the
    float32 product is narrowed (the reference's order) than when the exact
    product is rounded once: an implementation that fuses the multiply into
    the narrowing conversion fails on exactly these."""
    acc = np.arange(-442368, 442369, dtype=np.int64)
    s = np.float32(np.float32(gamma) * np.float32(absmax)) / np.float32(127.0)
    exact = acc.astype(np.float64) * np.float64(s)
    via32 = exact.astype(np.float32)
    if kind == "f16":
        diff = via32.astype(np.float16) != exact.astype(np.float16)
    else:
        import torch as T
        diff = (T.from_numpy(via32).to(T.bfloat16).float().numpy()
                != T.from_numpy(exact).to(T.bfloat16).float().numpy())
    return acc[diff].astype(np.int32)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_dequantize(gpu, kind):
    gamma, absmax = 0.8123, 3.37
    tricky = double_rounding_cases(gamma, absmax, kind)
    if kind == "f16":
        assert tricky.size > 10  # the check below has teeth
    rnd = np.random.default_rng(3).integers(-442368, 442369, 6912).astype(np.int32)
    acc = np.concatenate([np.array([0, 1, -1, 442368, -442368], np.int32), tricky, rnd])
    n = acc.size
    d_a = torch.tensor([absmax], dtype=torch.float32, device=gpu)
    out = torch.zeros(n, dtype=HALF[kind], device=gpu)
    K.dequantize_gpu(dev(acc, gpu), out, d_a, gamma, n)
    torch.cuda.synchronize()
    assert (half_bits(out) == oracle_half_bits(O.dequant(acc, gamma, absmax), kind)).all()


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("rows,cols", [(6912, 2560), (2560, 6912), (640, 2560), (96, 100)])
def test_fused_bitlinear(gpu, kind, rows, cols):
    L = W.random_layer(rows, cols, W.seed_for("fused", rows, cols))
    x, xf = half_tensor(W.normal_f32(W.seed_for("fx", rows, cols), cols), kind, gpu)
    d_a = torch.zeros(1, dtype=torch.float32, device=gpu)
    out = torch.zeros(rows, dtype=HALF[kind], device=gpu)
    K.absmax_reduce_gpu(x, d_a, cols)
    K.fused_sparse_bitlinear_gpu(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), x, out, d_a, L.gamma,
                                 rows, cols, L.meta_stride, L.values_stride)
    torch.cuda.synchronize()
    amax = O.absmax(xf)
    want, acc = O.fused_bitlinear(L.meta, L.values, xf, amax, L.gamma, rows, cols)
    # Bit-exact 16-bit outputs: stricter than the contract's 1e-3 relative bound.
    assert (half_bits(out) == oracle_half_bits(want, kind)).all()


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("rows,cols,shift", [(6912, 2560, 0), (2560, 6912, 0), (640, 2048, 0),
                                             (96, 100, 0), (300, 2560, 1)])
def test_one_call_bitlinear(gpu, kind, rows, cols, shift):
    """spb_bitlinear_* (InferenceEngine::bitlinear as one call, the absmax
    scratch and the activation planes in a caller workspace): output bits
    equal the oracle's fused BitLinear.  cols % 8 != 0 and an x that is not
    16-byte aligned (shift) take the reference's pair on the workspace's
    absmax instead of the planes."""
    L = W.random_layer(rows, cols, W.seed_for("bitlinear1", rows, cols))
    a = W.normal_f32(W.seed_for("bitlinear1-x", rows, cols), cols + shift)
    xt, xf = half_tensor(a, kind, gpu)
    x = xt[shift:]
    xf = xf[shift:]
    out = torch.zeros(rows, dtype=HALF[kind], device=gpu)
    ws = torch.full((K.bitlinear_workspace_size(cols),), 0xA5, dtype=torch.uint8, device=gpu)
    K.bitlinear_gpu(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), x, out, L.gamma, rows, cols,
                    L.meta_stride, L.values_stride, ws)
    torch.cuda.synchronize()
    want, _ = O.fused_bitlinear(L.meta, L.values, xf, O.absmax(xf), L.gamma, rows, cols)
    assert (half_bits(out) == oracle_half_bits(want, kind)).all()
