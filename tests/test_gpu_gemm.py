"""GPU parity of the batched GEMM (replacing the reference's cuSPARSELt path,
whose own test checks D = A_pruned * B exactly against cpu_int8_gemm,
tests/test_cusparselt.cu:16-28, 127-274) against the CPU oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from spbitnet_amd import kernels as K
from spbitnet_amd import weights as W
from tests.test_gpu_sparse_ternary import dev, dev_u32

pytestmark = pytest.mark.gpu


def expected(L, X):
    """Exact int32 product via the oracle's unpacked matrix (float64 BLAS is
    exact here: |products| <= 128 and |sums| < 2^53)."""
    dense = O.unpack(L.meta, L.values, L.rows, L.cols).astype(np.float64)
    return (X.astype(np.float64) @ dense.T).astype(np.int64).astype(np.int32)


def run(L, X, gpu, kernel="auto"):
    n = X.shape[0]
    Y = torch.full((n, L.rows), -7, dtype=torch.int32, device=gpu)
    K.sparse_ternary_gemm_gpu(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), dev(X, gpu), Y,
                              L.rows, L.cols, n, L.meta_stride, L.values_stride, kernel=kernel)
    torch.cuda.synchronize()
    return Y.cpu().numpy()


def activations(n, cols, seed):
    q = np.zeros((n, cols), np.int8)
    for t in range(n):
        q[t], _ = W.quantize_absmax_host(W.normal_f32(seed + t, cols))
    return q


def test_gemm_n16_matches_oracle_gemm(gpu):
    """cpu_int8_gemm (the oracle) at the reference test's shape family."""
    rows, cols, n = 64, 256, 16
    L = W.random_layer(rows, cols, 5)
    X = np.random.default_rng(6).integers(-5, 6, (n, cols)).astype(np.int8)
    assert (run(L, X, gpu) == O.gemm(L.meta, L.values, X, rows, cols)).all()


@pytest.mark.parametrize("n", [16, 64, 256])
def test_gemm_config2(gpu, n):
    rows, cols = 6912, 2560
    L = W.random_layer(rows, cols, W.seed_for("gemm", n))
    X = activations(n, cols, 1000 + n)
    X_dev = dev(X, gpu)
    assert K.gemm_kernel_id(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), X_dev, rows, cols, n,
                            L.meta_stride, L.values_stride) == 2
    assert (run(L, X, gpu) == expected(L, X)).all()


@pytest.mark.parametrize("rows,cols,n", [(2560, 6912, 16), (7, 128, 1), (333, 384, 5),
                                         (100, 256, 17), (16, 512, 100), (45, 100, 3),
                                         (9, 36, 20), (640, 2560, 200), (2560, 2560, 129),
                                         (6912, 2560, 1023), (1000, 1024, 300)])
def test_gemm_odd_shapes(gpu, rows, cols, n):
    L = W.random_layer(rows, cols, W.seed_for("gemm-odd", rows, cols, n))
    X = np.random.default_rng(rows + cols + n).integers(-128, 128, (n, cols)).astype(np.int8)
    assert (run(L, X, gpu) == expected(L, X)).all()


def test_gemm_extremes(gpu):
    rows, cols, n = 32, 6912, 16
    L = W.random_layer(rows, cols, 8)
    dense = O.unpack(L.meta, L.values, rows, cols)
    X = np.stack([np.full(cols, -128), np.full(cols, 127)] +
                 [np.where(dense[i] < 0, -128, 127) for i in range(14)]).astype(np.int8)
    assert (run(L, X, gpu) == expected(L, X)).all()


@pytest.mark.parametrize("n", [1, 16, 37])
def test_gemm_addsub_comparator(gpu, n):
    rows, cols = 2560, 2560
    L = W.random_layer(rows, cols, W.seed_for("addsub", n))
    X = activations(n, cols, 77)
    assert (run(L, X, gpu, kernel="addsub") == expected(L, X)).all()


@pytest.mark.parametrize("rows,cols,n", [(2560, 6912, 64), (2560, 6912, 256), (96, 768, 33),
                                         (48, 2816, 16), (200, 512, 70), (64, 256, 64)])
def test_gemm_partial_chunks_and_tiles(gpu, rows, cols, n):
    """Column counts whose last staged chunk is partial (6912 = 27 column
    pairs, 2816 = 11, 768 = 3), row counts that end inside a row block and
    batches that end inside a token tile."""
    L = W.random_layer(rows, cols, W.seed_for("gemm-chunks", rows, cols, n))
    X = np.random.default_rng(rows * 7 + cols + n).integers(-128, 128, (n, cols)).astype(np.int8)
    assert (run(L, X, gpu) == expected(L, X)).all()


@pytest.mark.parametrize("pad_m,pad_v", [(4, 4), (8, 0), (1, 0), (0, 2), (3, 5)])
@pytest.mark.parametrize("n", [16, 64, 200])
def test_gemm_padded_strides(gpu, pad_m, pad_v, n):
    """Row strides past the format's minimum: multiples of 4 words keep the
    staged matrix-core kernel, others take the direct one; both exact, and the
    padding words (all ones, invalid bitmaps) change nothing."""
    rows, cols = 160, 2560
    L = W.random_layer(rows, cols, W.seed_for("gemm-pad", pad_m, pad_v, n))
    meta = np.full((rows, L.meta_stride + pad_m), 0xFFFFFFFF, np.uint32)
    values = np.full((rows, L.values_stride + pad_v), 0xFFFFFFFF, np.uint32)
    meta[:, :L.meta_stride] = L.meta
    values[:, :L.values_stride] = L.values
    X = activations(n, cols, 500 + pad_m + pad_v)
    m_dev, v_dev, X_dev = dev_u32(meta, gpu), dev_u32(values, gpu), dev(X, gpu)
    staged = meta.shape[1] % 4 == 0 and values.shape[1] % 4 == 0
    assert K.gemm_kernel_id(m_dev, v_dev, X_dev, rows, cols, n, meta.shape[1],
                            values.shape[1]) == (2 if staged else 1)
    Y = torch.full((n, rows), -7, dtype=torch.int32, device=gpu)
    K.sparse_ternary_gemm_gpu(m_dev, v_dev, X_dev, Y, rows, cols, n, meta.shape[1],
                              values.shape[1])
    torch.cuda.synchronize()
    assert (Y.cpu().numpy() == expected(L, X)).all()


@pytest.mark.parametrize("rows,cols,n", [(333, 512, 5), (6, 256, 17), (2561, 2560, 100),
                                         (18, 768, 64), (1001, 2816, 33)])
def test_gemm_staged_rows_not_multiple_of_4(gpu, rows, cols, n):
    """The staged matrix-core kernel (kernel id 2) on row counts that are not a
    multiple of 4: each token's rows are stored one by one, so no token's
    rows overwrite the next token's and nothing lands past Y's end (checked
    with guard words after Y)."""
    L = W.random_layer(rows, cols, W.seed_for("gemm-rows4", rows, cols, n))
    X = np.random.default_rng(rows + 3 * cols + n).integers(-128, 128, (n, cols)).astype(np.int8)
    m_dev, v_dev, X_dev = dev_u32(L.meta, gpu), dev_u32(L.values, gpu), dev(X, gpu)
    assert K.gemm_kernel_id(m_dev, v_dev, X_dev, rows, cols, n, L.meta_stride,
                            L.values_stride) == 2
    guard = 64
    buf = torch.full((n * rows + guard,), -7, dtype=torch.int32, device=gpu)
    K.sparse_ternary_gemm_gpu(m_dev, v_dev, X_dev, buf, rows, cols, n, L.meta_stride,
                              L.values_stride)
    torch.cuda.synchronize()
    out = buf.cpu().numpy()
    assert (out[:n * rows].reshape(n, rows) == expected(L, X)).all()
    assert (out[n * rows:] == -7).all()


@pytest.mark.parametrize("rows,cols,n", [(6900, 2560, 250), (3333, 768, 500), (13824, 512, 129),
                                         (2560, 6912, 700), (6912, 2560, 256)])
def test_gemm_wide_128_row_tile(gpu, rows, cols, n):
    """Batches above 64 tokens whose 128-row x 64-token grid nearly fills the
    chip take the 128-row staged tile (one column pair per chunk): rows that
    end inside a row block or are not a multiple of 4, batches that end inside
    a token tile, 27-pair rows; exact, and nothing written past Y (guard
    words)."""
    L = W.random_layer(rows, cols, W.seed_for("gemm-wide128", rows, cols, n))
    X = np.random.default_rng(rows + 11 * cols + n).integers(-128, 128, (n, cols)).astype(np.int8)
    m_dev, v_dev, X_dev = dev_u32(L.meta, gpu), dev_u32(L.values, gpu), dev(X, gpu)
    assert K.gemm_kernel_id(m_dev, v_dev, X_dev, rows, cols, n, L.meta_stride,
                            L.values_stride) == 2
    guard = 64
    buf = torch.full((n * rows + guard,), -7, dtype=torch.int32, device=gpu)
    K.sparse_ternary_gemm_gpu(m_dev, v_dev, X_dev, buf, rows, cols, n, L.meta_stride,
                              L.values_stride)
    torch.cuda.synchronize()
    out = buf.cpu().numpy()
    assert (out[:n * rows].reshape(n, rows) == expected(L, X)).all()
    assert (out[n * rows:] == -7).all()


@pytest.mark.parametrize("rows,cols,n", [(256, 512, 20), (6912, 2560, 256)])
def test_gemm_staged_unaligned_output(gpu, rows, cols, n):
    """Y that starts 4 bytes past a 16-byte boundary (rows a multiple of 4):
    the staged kernel stores rows one by one instead of 16-byte quads (the
    32x16 tile, and the 128-row tile at 256 tokens)."""
    L = W.random_layer(rows, cols, W.seed_for("gemm-unaligned-y", rows, cols, n))
    X = np.random.default_rng(91).integers(-128, 128, (n, cols)).astype(np.int8)
    buf = torch.full((n * rows + 8,), -7, dtype=torch.int32, device=gpu)
    Y = buf[1:1 + n * rows]
    K.sparse_ternary_gemm_gpu(dev_u32(L.meta, gpu), dev_u32(L.values, gpu), dev(X, gpu), Y,
                              rows, cols, n, L.meta_stride, L.values_stride)
    torch.cuda.synchronize()
    out = buf.cpu().numpy()
    assert out[0] == -7 and (out[1 + n * rows:] == -7).all()
    assert (out[1:1 + n * rows].reshape(n, rows) == expected(L, X)).all()


@pytest.mark.parametrize("rows,cols,n", [(640, 2560, 40), (3840, 2560, 32), (100, 1024, 50),
                                         (130, 2304, 17), (64, 256, 64), (6912, 2560, 64)])
def test_gemm_n17_to_64_tiles(gpu, rows, cols, n):
    """17-64 tokens (the 64-row x 32-token staged tile) on rows of at most
    2560 columns: full and partial column pairs, rows that end inside a row
    block, batches that end inside a token tile."""
    L = W.random_layer(rows, cols, W.seed_for("gemm-n17-64", rows, cols, n))
    X = np.random.default_rng(rows + 5 * cols + n).integers(-128, 128, (n, cols)).astype(np.int8)
    assert (run(L, X, gpu) == expected(L, X)).all()
