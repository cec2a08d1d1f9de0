"""GPU parity of the bit-plane activation entry points (no reference
counterpart: they produce and consume an activation layout of this build)
against the oracle's layout definition and the int8 / fused entry points."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from spbitnet_amd import kernels as K
from spbitnet_amd import weights as W
from tests.test_gpu_sparse_ternary import (CONFIG_SHAPES, HALF, dev, dev_u32, half_bits,
                                           half_tensor, oracle_half_bits, quantized_activation)

pytestmark = pytest.mark.gpu


def planes_to_numpy(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("cols", [8, 64, 96, 2560, 6912, 2568, 32768])
def test_activation_planes_layout(gpu, cols):
    x = np.random.default_rng(cols).integers(-128, 128, cols).astype(np.int8)
    planes = torch.full((K.planes_words(cols),), -1, dtype=torch.int32, device=gpu)
    K.activation_planes_gpu(dev(x, gpu), planes, cols)
    torch.cuda.synchronize()
    assert (planes_to_numpy(planes) == O.planes(x)).all()


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("n", [8, 2560, 6912])
def test_absmax_quantize_planes(gpu, kind, n):
    x, xf = half_tensor(W.normal_f32(W.seed_for("qp", n), n) * 2, kind, gpu)
    planes = torch.full((K.planes_words(n),), -1, dtype=torch.int32, device=gpu)
    q = torch.zeros(n, dtype=torch.int8, device=gpu)
    d_a = torch.zeros(1, dtype=torch.float32, device=gpu)
    K.absmax_quantize_planes_gpu(x, planes, d_a, n, output=q)
    torch.cuda.synchronize()
    oq, oa = O.quantize(xf)
    assert d_a.item() == oa
    assert (q.cpu().numpy() == oq).all()
    assert (planes_to_numpy(planes) == O.planes(oq)).all()


@pytest.mark.parametrize("rows,cols", CONFIG_SHAPES + [(7, 256), (333, 384), (64, 100), (9, 36)])
def test_gemv_planes_matches_oracle(gpu, rows, cols):
    L = W.random_layer(rows, cols, W.seed_for("gp", rows, cols))
    x = quantized_activation(cols, W.seed_for("gpx", rows, cols), relu2=(cols > rows))
    planes = torch.from_numpy(O.planes(x).view(np.int32)).to(gpu)
    y = torch.full((rows,), -7, dtype=torch.int32, device=gpu)
    K.sparse_ternary_gemv_planes_gpu(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), planes, y,
                                     rows, cols, L.meta_stride, L.values_stride)
    torch.cuda.synchronize()
    assert (y.cpu().numpy() == O.gemv(L.meta, L.values, x, rows, cols)).all()


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("rows,cols", [(6912, 2560), (2560, 6912), (96, 96)])
def test_fused_bitlinear_planes(gpu, kind, rows, cols):
    L = W.random_layer(rows, cols, W.seed_for("fp", rows, cols))
    x, xf = half_tensor(W.normal_f32(W.seed_for("fpx", rows, cols), cols), kind, gpu)
    planes = torch.zeros(K.planes_words(cols), dtype=torch.int32, device=gpu)
    d_a = torch.zeros(1, dtype=torch.float32, device=gpu)
    out = torch.zeros(rows, dtype=HALF[kind], device=gpu)
    K.absmax_quantize_planes_gpu(x, planes, d_a, cols)
    K.fused_sparse_bitlinear_planes_gpu(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), planes, out,
                                        d_a, L.gamma, rows, cols, L.meta_stride, L.values_stride)
    torch.cuda.synchronize()
    want, _ = O.fused_bitlinear(L.meta, L.values, xf, O.absmax(xf), L.gamma, rows, cols)
    assert (half_bits(out) == oracle_half_bits(want, kind)).all()
