"""GPU parity of the structured-sparse int8 GEMM, the drop-in for the
reference's cuSPARSELt backend (CuSparseLtGemm, include/spbitnet/
cusparselt_backend.h:28-77): the reference's own tests
(tests/test_cusparselt.cu:68-274: the pruned matrix is 2:4 with values from
A, and D = A_pruned * B exactly against cpu_int8_gemm) restated, plus the
config-2 shapes, odd shapes, full-range int8 values and the C++ mirror."""
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spbitnet_amd import _lib
from spbitnet_amd import kernels as K

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(A, B, gpu):
    """(D [n][m], pruned [m][k]) from the Python mirror of CuSparseLtGemm."""
    m, k = A.shape
    n = B.shape[0]
    ctx = K.CuSparseLtGemm(m, k, n, device=gpu)
    dA = torch.from_numpy(A).to(gpu)
    dB = torch.from_numpy(np.ascontiguousarray(B)).to(gpu)
    D = torch.full((n, m), -7, dtype=torch.int32, device=gpu)
    P = torch.full((m, k), 99, dtype=torch.int8, device=gpu)
    ctx.prepare(dA)
    ctx.execute(dB, D)
    ctx.get_pruned_weights(P)
    torch.cuda.synchronize()
    return D.cpu().numpy(), P.cpu().numpy(), ctx.kernel_id(dB)


def _exact(Pr, B):
    """D [n][m] = B Pr^T, exact in float64 (|sums| < 2^53)."""
    return (B.astype(np.float64) @ Pr.astype(np.float64).T).astype(np.int64).astype(np.int32)


def test_prune_produces_24_pattern(gpu):
    """tests/test_cusparselt.cu:68-117: values {-1,0,1}, m=64, k=256."""
    A = np.random.default_rng(42).integers(-1, 2, (64, 256)).astype(np.int8)
    B = np.zeros((16, 256), np.int8)
    _, P, _ = _run(A, B, gpu)
    assert ((P >= -1) & (P <= 1)).all()
    assert ((P.reshape(64, -1, 4) != 0).sum(-1) <= 2).all()
    assert (P == 0).mean() >= 0.45
    assert np.array_equal(P, O.prune24_i8(A))
    assert K.sparse_i8_prune_check(torch.from_numpy(P).to(gpu), 64, 256) == 0
    bad = int((((A.reshape(64, -1, 4) != 0).sum(-1)) > 2).sum())
    assert bad > 0 and K.sparse_i8_prune_check(torch.from_numpy(A).to(gpu), 64, 256) == bad


def test_gemm_n16_correctness(gpu):
    """tests/test_cusparselt.cu:123-201: m=64, k=256, n=16, B in [-5, 5]."""
    rng = np.random.default_rng(123)
    A = rng.integers(-1, 2, (64, 256)).astype(np.int8)
    B = rng.integers(-5, 6, (16, 256)).astype(np.int8)
    D, P, kid = _run(A, B, gpu)
    assert kid == 1
    assert np.array_equal(P, O.prune24_i8(A))
    assert np.array_equal(D, O.int8_gemm(P, B))


def test_gemm_large_dimension(gpu):
    """tests/test_cusparselt.cu:206-274 (2048 x 2048, n = 32), every row
    checked (the reference checks 64)."""
    rng = np.random.default_rng(99)
    A = rng.integers(-1, 2, (2048, 2048)).astype(np.int8)
    B = rng.integers(-5, 6, (32, 2048)).astype(np.int8)
    D, P, _ = _run(A, B, gpu)
    assert np.array_equal(P, O.prune24_i8(A))
    assert np.array_equal(D, _exact(P, B))
    assert np.array_equal(D[:, :64], O.int8_gemm(P[:64], B))


@pytest.mark.parametrize("n", [1, 16, 64, 256])
def test_config2_shape_full_range(gpu, n):
    """6912 x 2560 (the FFN shape of config 2) with int8 values over the whole
    range in A and B: exact int32 products."""
    rng = np.random.default_rng(1000 + n)
    A = rng.integers(-128, 128, (6912, 2560)).astype(np.int8)
    B = rng.integers(-128, 128, (n, 2560)).astype(np.int8)
    D, P, kid = _run(A, B, gpu)
    assert kid == 1
    assert np.array_equal(P, O.prune24_i8(A))
    assert np.array_equal(D, _exact(P, B))


@pytest.mark.parametrize("m,k,n", [(1, 16, 1), (17, 144, 3), (100, 272, 33), (333, 1040, 70),
                                   (2560, 6912, 20), (48, 4, 5), (21, 100, 9), (5, 36, 65)])
def test_odd_shapes(gpu, m, k, n):
    """Rows that end inside a 16-row strip, columns that end inside a
    128-column step, k % 16 != 0 (the general kernel) and batches that end
    inside a token tile."""
    rng = np.random.default_rng(m * 31 + k * 7 + n)
    A = rng.integers(-128, 128, (m, k)).astype(np.int8)
    B = rng.integers(-128, 128, (n, k)).astype(np.int8)
    D, P, kid = _run(A, B, gpu)
    assert kid == (1 if k % 16 == 0 else 0)
    assert np.array_equal(P, O.prune24_i8(A))
    assert np.array_equal(D, O.int8_gemm(P, B))


def test_unaligned_b_takes_general_kernel(gpu):
    m, k, n = 64, 256, 17
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, (m, k)).astype(np.int8)
    B = rng.integers(-128, 128, (n, k)).astype(np.int8)
    ctx = K.CuSparseLtGemm(m, k, n, device=gpu)
    ctx.prepare(torch.from_numpy(A).to(gpu))
    buf = torch.zeros(n * k + 16, dtype=torch.int8, device=gpu)
    buf[3:3 + n * k] = torch.from_numpy(B.ravel()).to(gpu)
    dB = buf[3:3 + n * k]
    assert ctx.kernel_id(dB) == 0
    D = torch.empty((n, m), dtype=torch.int32, device=gpu)
    ctx.execute(dB, D)
    torch.cuda.synchronize()
    assert np.array_equal(D.cpu().numpy(), O.int8_gemm(O.prune24_i8(A), B))


def test_already_24_matrix_is_unchanged_and_extremes(gpu):
    """A matrix with at most two non-zeros per group (including the -128 /
    127 extremes) is kept as it is; products reach |D| = 128 * 128 * k / 2."""
    m, k, n = 96, 2560, 48
    rng = np.random.default_rng(6)
    A = rng.integers(-128, 128, (m, k)).astype(np.int8)
    g = A.reshape(m, -1, 4)
    drop = rng.integers(0, 4, g.shape[:2])
    for d in range(4):
        g[..., d][(drop == d) | (drop == (d + 1) % 4)] = 0
    A = g.reshape(m, k)
    A[0] = np.tile(np.array([-128, 0, -128, 0], np.int8), k // 4)
    A[1] = np.tile(np.array([0, 127, 0, 127], np.int8), k // 4)
    B = rng.integers(-128, 128, (n, k)).astype(np.int8)
    B[0] = -128
    D, P, _ = _run(A, B, gpu)
    assert np.array_equal(P, A)
    assert np.array_equal(D, _exact(A, B))
    assert D[0, 0] == 128 * 128 * (k // 2)


def test_bad_input_rejected(gpu):
    with pytest.raises(_lib.SpbError, match="multiple of 4"):
        K.CuSparseLtGemm(16, 6, 16, device=gpu)
    ctx = K.CuSparseLtGemm(16, 64, 16, device=gpu)
    with pytest.raises(RuntimeError, match="before prepare"):
        ctx.execute(torch.zeros((16, 64), dtype=torch.int8, device=gpu),
                    torch.zeros((16, 16), dtype=torch.int32, device=gpu))


def test_cpp_mirror_program(gpu, tmp_path):
    """The reference's call sequence (construct, prepare, execute,
    get_pruned_weights) in a C++ host program against
    include/spbitnet/cusparselt_backend.h, with the reference test's
    column-major B and D."""
    exe = os.path.join(ROOT, "tests", "cpp", "cusparselt_api")
    assert os.path.exists(exe), "tests/cpp/cusparselt_api is not built"
    m, k, n = 640, 2560, 16
    rng = np.random.default_rng(77)
    A = rng.integers(-1, 2, (m, k)).astype(np.int8)
    B = rng.integers(-5, 6, (n, k)).astype(np.int8)  # [n][k] = column-major [k x n]
    A.tofile(tmp_path / "A.bin")
    B.tofile(tmp_path / "B.bin")
    print("running the C++ cuSPARSELt-backend program", flush=True)
    r = subprocess.run([exe, str(tmp_path), str(m), str(k), str(n)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert f"m {m} k {k} n {n}" in r.stdout
    P = np.fromfile(tmp_path / "pruned.bin", dtype=np.int8).reshape(m, k)
    D = np.fromfile(tmp_path / "D.bin", dtype=np.int32).reshape(n, m)  # column-major [m x n]
    assert np.array_equal(P, O.prune24_i8(A))
    assert np.array_equal(D, O.int8_gemm(P, B))
