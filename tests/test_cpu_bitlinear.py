"""The PyTorch CPU BitLinear restatement (oracle/cpu_bitlinear.py, after
python/baseline_pytorch.py:56-107) that bench.py times as a CPU baseline,
pinned against the C oracle: its float32 matmul accumulators are the exact
int32 GEMV of the quantised input (a plausible slip such as a transposed
weight or a dropped clamp changes them), and its fp16 output is within the
contract's 1e-3 relative bound of the oracle's fused BitLinear (the Python
float64 dequant scale differs from the kernels' float32 order by rounding
only)."""
import numpy as np
import torch

from oracle import oracle as O
from oracle.cpu_bitlinear import TorchSparseBitLinear
from spbitnet_amd import weights as W


def test_torch_bitlinear_matches_oracle():
    for rows, cols in [(640, 2560), (96, 256), (256, 1024)]:
        L = W.random_layer(rows, cols, W.seed_for("torch-bl", rows, cols))
        a = W.normal_f32(W.seed_for("torch-bl-x", rows, cols), cols) * 2.0
        x16 = torch.from_numpy(a).half()
        xf = x16.float().numpy()
        m = TorchSparseBitLinear(L.meta, L.values, L.gamma, rows, cols)
        q, amax = O.quantize(xf)
        acc = O.gemv(L.meta, L.values, q, rows, cols)
        assert np.array_equal(m.accumulators(x16).numpy().astype(np.int64), acc.astype(np.int64))
        want, acc2 = O.fused_bitlinear(L.meta, L.values, xf, O.absmax(xf), L.gamma, rows, cols)
        assert np.array_equal(acc, acc2)
        got = m(x16).float().numpy()
        w16 = want.astype(np.float16).astype(np.float32)
        assert np.all(np.abs(got - w16) <= 1e-3 * np.abs(w16) + 1e-6)


def test_torch_bitlinear_zero_input():
    L = W.random_layer(64, 256, 3)
    m = TorchSparseBitLinear(L.meta, L.values, L.gamma, 64, 256)
    assert (m(torch.zeros(256, dtype=torch.float16)) == 0).all()


def test_dense_mac_is_the_gemv_without_unpack():
    L = W.random_layer(128, 512, 5)
    x = np.random.default_rng(1).integers(-128, 128, 512).astype(np.int8)
    dense = O.unpack(L.meta, L.values, 128, 512)
    assert np.array_equal(O.dense_mac(dense, x), O.gemv(L.meta, L.values, x, 128, 512))
