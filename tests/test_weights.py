"""Host-side format code of the product (spbitnet_amd/weights.py) against the
pinned oracle and, where built, the reference's own format code."""
import numpy as np
import pytest

from oracle import oracle as O
from spbitnet_amd import weights as W


@pytest.mark.parametrize("rows,cols", [(1, 4), (3, 36), (8, 64), (17, 100), (64, 256), (40, 2560)])
def test_packer_matches_oracle(rows, cols):
    w = W.normal_f32(W.seed_for("pack", rows, cols), rows * cols).reshape(rows, cols)
    m = W.top2_mask(w)
    assert (m == O.mask_top2(w).astype(bool)).all()
    dense = W.ternary_sparse(w, m)
    assert (dense == O.kept_sign(w, m.astype(np.uint8))).all()
    meta, values = W.pack(dense, m)
    om, ov = O.pack(dense, m.astype(np.uint8))
    assert (meta == om).all() and (values == ov).all()
    assert (W.unpack(meta, values, rows, cols) == dense).all()
    if O.ref_available():
        rm, rv = O.ref_pack_from_dense(dense, m.astype(np.uint8))
        assert (meta == rm).all() and (values == rv).all()


def test_mask_ties_follow_stable_argsort():
    w = np.array([[1, 1, 1, 1, 0.5, -0.5, 0.2, 0.5, 0, 0, 0, 0, 3, -3, 3, 1]], np.float32)
    assert (W.top2_mask(w) == O.mask_top2(w).astype(bool)).all()
    assert W.top2_mask(w)[0, :4].tolist() == [False, False, True, True]


def test_pack_rejects_bad_masks():
    with pytest.raises(ValueError):
        W.pack(np.ones((1, 6), np.int8), np.ones((1, 6), bool))
    with pytest.raises(ValueError):
        W.pack(np.ones((1, 4), np.int8), np.array([[1, 1, 1, 0]], bool))


def test_kept_zero_encodes_as_plus_one():
    dense = np.array([[0, 0, -1, 0]], np.int8)
    mask = np.array([[1, 0, 1, 0]], bool)
    meta, values = W.pack(dense, mask)
    assert meta[0, 0] == 0x5 and values[0, 0] == 0b10
    if O.ref_available():
        rm, rv = O.ref_pack_from_dense(dense, mask.astype(np.uint8))
        assert rm[0, 0] == meta[0, 0] and rv[0, 0] == values[0, 0]


def test_generator_deterministic_and_normal():
    a = W.normal_f32(123, 200001)
    b = W.normal_f32(123, 200001)
    assert (a == b).all() and a.dtype == np.float32
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1) < 0.01
    # chunking does not change the stream
    c = W.normal_f32(123, 200001, chunk=777)
    assert (a == c).all()
    assert not (W.normal_f32(124, 1000) == a[:1000]).all()


def test_compression_ratio_kat(kat):
    k = kat["compression_ratio"]
    rows, cols = k["rows"], k["cols"]
    dense = np.ones((rows, cols), np.int8)
    mask = np.tile(np.array([1, 1, 0, 0], bool), (rows, cols // 4))
    meta, values = W.pack(dense, mask)
    dense_2bit_bytes = rows * ((cols + 15) // 16) * 4
    ratio = (meta.nbytes + values.nbytes) / dense_2bit_bytes
    assert k["lo"] < ratio < k["hi"]


def test_random_layer_shapes_and_gamma():
    L = W.random_layer(64, 256, 7)
    assert L.meta.shape == (64, 8) and L.values.shape == (64, 4)
    w = W.normal_f32(7, 64 * 256)
    # the converter's gamma = float(np.mean(np.abs(weights))) on the float32
    # latent (convert_model.py:132): the same bits, not just the same value
    assert L.gamma == float(np.mean(np.abs(w.reshape(64, 256))))
    assert np.float32(L.gamma) == np.float32(np.mean(np.abs(w), dtype=np.float32))
    assert L.nbytes() == 64 * 256 * 3 // 16


def test_host_quantizer_matches_oracle():
    x = W.normal_f32(99, 2560)
    q, a = W.quantize_absmax_host(x)
    oq, oa = O.quantize(x)
    assert (q == oq).all() and a == oa
