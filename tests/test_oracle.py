"""Pins the CPU oracle (oracle/spb_oracle.c) before anything is checked
against it: the reference's known-answer tests, golden vectors regenerated
from the reference's own tests, the reference's own format code built into
oracle/_ref, and closed forms / library routines the semantics reduce to.
Each block also plants a plausible mistake in a CPU copy of the oracle's
result and shows the check rejects it."""
import hashlib
import itertools

import numpy as np
import pytest

from oracle import oracle as O


def _group(vals):
    return np.array([vals], np.float32)


# ---- format: strides, KATs, golden vectors ---------------------------------

def test_strides_match_formula_and_reference():
    for cols in [4, 8, 28, 32, 36, 64, 100, 128, 2048, 2560, 5632, 6912]:
        g = cols // 4
        assert O.meta_stride(cols) == (g + 7) // 8
        assert O.values_stride(cols) == (g + 15) // 16
        if O.ref_available():
            assert O.meta_stride(cols) == O.ref().ref_meta_stride(cols)
            assert O.values_stride(cols) == O.ref().ref_values_stride(cols)


def test_worked_example_kat(kat):
    k = kat["worked_example"]
    w = np.array([k["group"]], np.int8)
    m = (w != 0).astype(np.uint8)
    meta, values = O.pack(w, m)
    assert meta[0, 0] == k["bitmap"] and values[0, 0] == k["signs"]
    assert (O.unpack(meta, values, 1, 4) == w).all()
    # planted mistake: signs stored highest-first would give 0b01
    assert values[0, 0] != 0b01


def test_loader_pattern_kat(kat):
    k = kat["loader_pattern"]
    w = np.tile(np.array(k["group"], np.int8), (3, k["cols"] // 4))
    m = (w != 0).astype(np.uint8)
    meta, values = O.pack(w, m)
    assert (meta[:, 0] == k["meta_word"]).all()
    assert (values[:, 0] == k["values_word"]).all()


def test_pack_with_pruning_kat(kat):
    """The KAT's kept magnitudes are all > 0.5 with no ties, so the
    convert_model.py recipe the oracle follows gives the reference's answer."""
    k = kat["pack_with_pruning"]
    lat = np.array(k["latent"], np.float32)
    m = O.mask_top2(lat)
    dense = O.kept_sign(lat, m)
    meta, values = O.pack(dense, m)
    assert (O.unpack(meta, values, 2, 8) == np.array(k["expected"])).all()


def test_golden_roundtrip_and_unpack(golden, kat):
    for tag, rows, cols in [("roundtrip4x32", 4, 32)]:
        dense = golden[f"{tag}_dense"]
        m = (dense != 0).astype(np.uint8)
        meta, values = O.pack(dense, m)
        assert (meta == golden[f"{tag}_meta"]).all() and (values == golden[f"{tag}_values"]).all()
        assert (dense.reshape(rows, -1, 4) == np.array(kat["roundtrip"]["expected_group"])).all()
    w, m = golden["unpack8x64_w"], golden["unpack8x64_mask"]
    meta, values = O.pack(w, m)
    assert (meta == golden["unpack8x64_meta"]).all()
    assert (values == golden["unpack8x64_values"]).all()
    assert (O.unpack(meta, values, 8, 64) == golden["unpack8x64_dense"]).all()


def test_golden_gemv_64x256(golden):
    y = O.gemv(golden["gemv64x256_meta"], golden["gemv64x256_values"], golden["gemv64x256_x"], 64, 256)
    assert (y == golden["gemv64x256_y"]).all()
    # planted mistake: sign bits applied to the wrong kept column
    v = golden["gemv64x256_values"]
    swapped = ((v & 0x55555555) << 1) | ((v >> 1) & 0x55555555)
    y_bad = O.gemv(golden["gemv64x256_meta"], swapped.astype(np.uint32), golden["gemv64x256_x"], 64, 256)
    assert (y_bad != golden["gemv64x256_y"]).any()


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference tree absent)")
def test_golden_gemv_2048(golden):
    w, m, x = O.ref_make_test_case(77, 2048, 2048, True)
    meta, values = O.pack(w, m)
    h = hashlib.sha256(meta.tobytes() + values.tobytes()).digest()
    assert h == golden["gemv2048_meta_values_sha256"].tobytes()
    assert (x == golden["gemv2048_x"]).all()
    assert (O.gemv(meta, values, x, 2048, 2048) == golden["gemv2048_y"]).all()


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference tree absent)")
def test_oracle_matches_reference_format_code():
    rng = np.random.default_rng(5)
    for rows, cols in [(3, 4), (5, 36), (7, 100), (16, 256), (9, 2564)]:
        w = rng.integers(-1, 2, (rows, cols)).astype(np.int8)
        m = np.zeros((rows, cols), np.uint8)
        for r in range(rows):
            for g in range(cols // 4):
                m[r, 4 * g + rng.choice(4, 2, replace=False)] = 1
        meta, values = O.pack(w, m)
        rm, rv = O.ref_pack_from_dense(w, m)
        assert (meta == rm).all() and (values == rv).all()
        assert (O.unpack(meta, values, rows, cols) == O.ref_unpack(rm, rv, rows, cols)).all()


# ---- generator semantics (python/convert_model.py:88-138, 270-286) ----------

def _mask_by_stable_argsort(w):
    """The reference's own formulation, evaluated with numpy."""
    rows, cols = w.shape
    g = np.abs(w).reshape(rows, cols // 4, 4)
    order = np.argsort(g, axis=-1, kind="stable")[..., -2:]
    m = np.zeros_like(g, dtype=np.uint8)
    np.put_along_axis(m, order, 1, axis=-1)
    return m.reshape(rows, cols)


def test_mask_brute_force_all_orderings_and_ties():
    groups = []
    for perm in itertools.permutations([0.1, 0.2, 0.3, 0.4]):
        for signs in itertools.product([1, -1], repeat=4):
            groups.append([p * s for p, s in zip(perm, signs)])
    for pattern in itertools.product([0.0, 0.5, 1.0], repeat=4):  # many ties
        groups.append(list(pattern))
        groups.append([-v for v in pattern])
    w = np.array(groups, np.float32).reshape(1, -1)
    assert (O.mask_top2(w) == _mask_by_stable_argsort(w)).all()
    # ties go to the higher index
    assert (O.mask_top2(_group([1, 1, 1, 1])) == [[0, 0, 1, 1]]).all()
    assert (O.mask_top2(_group([2, 1, 1, 1])) == [[1, 0, 0, 1]]).all()
    # planted mistake: lower-index tie break (pack_with_pruning's rule) differs
    assert not (O.mask_top2(_group([1, 1, 1, 1])) == [[1, 1, 0, 0]]).all()


def test_kept_sign_is_gamma_independent():
    w = _group([-0.3, 0.2, -0.0, 0.0])
    m = np.ones_like(w, np.uint8)
    assert (O.kept_sign(w, m) == [[-1, 1, 1, 1]]).all()
    # RoundClip(w/gamma) then the zero-at-mask fix (convert_model.py:281-283)
    rng = np.random.default_rng(1)
    w = rng.standard_normal((4, 64)).astype(np.float32)
    m = O.mask_top2(w).astype(bool)
    gamma = np.float32(np.mean(np.abs(w)))
    tern = np.clip(np.round(w / gamma), -1, 1).astype(np.int8) * m
    zero = m & (tern == 0)
    tern[zero & (w >= 0)] = 1
    tern[zero & (w < 0)] = -1
    assert (O.kept_sign(w, m.astype(np.uint8)) == tern).all()


def test_absmean_matches_numpy():
    w = np.random.default_rng(2).standard_normal(100000).astype(np.float32)
    assert abs(O.absmean(w) - float(np.mean(np.abs(w)))) < 1e-6


# ---- GEMV / GEMM closed forms ------------------------------------------------

def _random_packed(rows, cols, seed):
    rng = np.random.default_rng(seed)
    lat = rng.standard_normal((rows, cols)).astype(np.float32)
    m = O.mask_top2(lat)
    dense = O.kept_sign(lat, m)
    meta, values = O.pack(dense, m)
    return dense, meta, values


def test_gemv_closed_forms():
    rows, cols = 24, 96
    dense, meta, values = _random_packed(rows, cols, 3)
    ones = np.ones(cols, np.int8)
    assert (O.gemv(meta, values, ones, rows, cols) == dense.sum(1)).all()  # row sign sum
    for j in [0, 1, 5, 95]:
        e = np.zeros(cols, np.int8)
        e[j] = 1
        assert (O.gemv(meta, values, e, rows, cols) == dense[:, j]).all()  # column read-out
    # bitmap 0x3 / signs 0b10 everywhere: y = sum_g x[4g] - x[4g+1]
    meta3 = np.full((2, O.meta_stride(cols)), 0x33333333, np.uint32)
    val2 = np.full((2, O.values_stride(cols)), 0xAAAAAAAA, np.uint32)
    x = np.random.default_rng(4).integers(-128, 128, cols).astype(np.int8)
    expect = int(x[0::4].astype(np.int64).sum() - x[1::4].astype(np.int64).sum())
    assert (O.gemv(meta3, val2, x, 2, cols) == expect).all()
    # linearity in x
    x1 = np.random.default_rng(6).integers(-64, 64, cols).astype(np.int8)
    x2 = np.random.default_rng(7).integers(-64, 64, cols).astype(np.int8)
    assert (O.gemv(meta, values, (x1 + x2).astype(np.int8), rows, cols)
            == O.gemv(meta, values, x1, rows, cols) + O.gemv(meta, values, x2, rows, cols)).all()


def test_gemm_is_batched_gemv():
    rows, cols, n = 16, 64, 5
    dense, meta, values = _random_packed(rows, cols, 8)
    X = np.random.default_rng(9).integers(-128, 128, (n, cols)).astype(np.int8)
    Y = O.gemm(meta, values, X, rows, cols)
    assert Y.shape == (n, rows)
    for t in range(n):
        assert (Y[t] == O.gemv(meta, values, X[t], rows, cols)).all()
    assert (Y == (X.astype(np.int64) @ dense.T.astype(np.int64))).all()


def test_accumulator_extremes_fit_int32():
    rows, cols = 2, 6912
    dense, meta, values = _random_packed(rows, cols, 10)
    x = np.where(dense[0] < 0, -128, 127).astype(np.int8)
    y = O.gemv(meta, values, x, rows, cols)
    assert y[0] == int(np.abs(dense[0]).astype(np.int64) @ np.where(dense[0] < 0, 128, 127))


# ---- quantisation / dequantisation ------------------------------------------

def test_quantize_closed_form():
    rng = np.random.default_rng(11)
    x = rng.standard_normal(6912).astype(np.float32)
    q, amax = O.quantize(x)
    assert amax == np.float32(np.max(np.abs(x)))
    scale = np.float32(127.0) / np.float32(amax)
    expect = np.clip(np.rint(x * scale), -128, 127).astype(np.int8)
    assert (q == expect).all()
    assert q.max() == 127 or q.min() == -127  # the absmax element maps to +-127


def test_quantize_zero_and_ties():
    q, amax = O.quantize(np.zeros(64, np.float32))
    assert amax == 0.0 and (q == 0).all()
    # absmax 127 -> scale exactly 1: half-way values round to even
    x = np.array([127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5], np.float32)
    q, _ = O.quantize(x)
    assert list(q) == [127, 0, 2, 2, 0, -2, -2, 4]
    # planted mistake: round-half-away-from-zero would give 1 for 0.5
    assert q[1] != 1


def test_dequant_float32_order():
    acc = np.array([0, 1, -1, 12345, -442368], np.int32)
    g, a = 0.8123, 3.7
    out = O.dequant(acc, g, a)
    s = np.float32(np.float32(g) * np.float32(a)) / np.float32(127.0)
    assert (out == acc.astype(np.float32) * np.float32(s)).all()


def test_fused_equals_quantize_gemv_dequant():
    rows, cols = 32, 256
    dense, meta, values = _random_packed(rows, cols, 12)
    x = np.random.default_rng(13).standard_normal(cols).astype(np.float32)
    q, amax = O.quantize(x)
    out, acc = O.fused_bitlinear(meta, values, x, amax, 0.77, rows, cols)
    assert (acc == O.gemv(meta, values, q, rows, cols)).all()
    assert (out == O.dequant(acc, 0.77, amax)).all()


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(14)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, 3.0e38, 1 + 2 ** -8, 1 + 3 * 2 ** -8],
                                 np.float32)])
    ours = O.to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (ours == ref).all()
    nan = O.to_bf16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


# ---- bit-plane activation layout (this build's own format) -------------------

def test_planes_round_trip_and_identity():
    rng = np.random.default_rng(15)
    for cols in [8, 40, 64, 2560, 6912]:
        x = rng.integers(-128, 128, cols).astype(np.int8)
        p = O.planes(x)
        assert p.size == 8 * ((cols + 31) // 32)
        words = p.reshape(-1, 8)
        back = np.zeros(cols, np.int64)
        for c in range(cols):
            v = sum(((int(words[c // 32, b]) >> (c % 32)) & 1) << b for b in range(8))
            back[c] = v - 256 if v >= 128 else v
        assert (back == x).all()
    # sum_j w_j x_j = sum_b c_b sum_j w_j bit_b(x_j), c_7 = -128
    dense, meta, values = _random_packed(8, 64, 16)
    x = rng.integers(-128, 128, 64).astype(np.int8)
    bits = ((x.astype(np.int64)[None, :] & 0xFF) >> np.arange(8)[:, None]) & 1
    c = np.array([1, 2, 4, 8, 16, 32, 64, -128])
    assert (dense.astype(np.int64) @ (c @ bits) == O.gemv(meta, values, x, 8, 64)).all()


# ---- the random-init model generator's host restatement (spb_gen.c) ----------

def test_generator_ln_sqrt_cos_match_libm():
    """The add/multiply-only ln, sqrt and cos of the generator against libm
    (float64), over the generator's whole input ranges' edges and random
    points: within 1e-14 relative (ln, sqrt) and 1e-15 absolute (cos)."""
    import math
    L = O.lib()
    rng = np.random.default_rng(5)
    ks = [1, 2, 3, 1 << 23, (1 << 23) + 1, (1 << 24) - 1, 1 << 24, 11863283, 11863284]
    ks += [int(k) for k in rng.integers(1, (1 << 24) + 1, 20000)]
    for k in ks:
        want = math.log(k / 2.0 ** 24)
        got = L.spbo_gen_ln_u24(k)
        assert abs(got - want) <= 1e-14 * abs(want), k
    js = [0, 1, (1 << 21) - 1, 1 << 21, (1 << 21) + 1, 1 << 22, (1 << 22) + 1, 1 << 23,
          (1 << 23) + 1, (1 << 24) - 1] + [int(j) for j in rng.integers(0, 1 << 24, 20000)]
    for j in js:
        assert abs(L.spbo_gen_cos_u24(j) - math.cos(2 * math.pi * j / 2.0 ** 24)) <= 1e-15, j
    for y in [0.0, 1e-8, 0.5, 1.0, 2.0, 33.27] + list(rng.uniform(0, 34, 5000)):
        want = math.sqrt(y)
        assert abs(L.spbo_gen_sqrt(y) - want) <= 1e-15 * max(want, 1e-300), y
    # u1 = 1 gives radius 0; cos at the octant edges is exact where it must be
    assert L.spbo_gen_ln_u24(1 << 24) == 0.0 and L.spbo_gen_sqrt(0.0) == 0.0
    assert L.spbo_gen_cos_u24(0) == 1.0 and L.spbo_gen_cos_u24(1 << 23) == -1.0


def test_generator_normals_are_standard_normal_and_deterministic():
    x = O.gen_normals(2025, 4_000_000)
    assert np.array_equal(x, O.gen_normals(2025, 4_000_000))
    assert np.array_equal(x[1000:1100], O.gen_normals(2025, 100, start=1000))
    assert abs(x.mean()) < 3e-3 and abs(x.std() - 1) < 2e-3
    assert abs(np.abs(x).mean() - np.sqrt(2 / np.pi)) < 2e-3
    assert abs((x.astype(np.float64) ** 4).mean() - 3) < 0.03
    # every float equals the float64 Box-Muller value rounded once (a wrong
    # branch of the cos reduction or a dropped log term would not)
    import math
    z = O.gen_normals(77, 2000)
    M = 0xFFFFFFFFFFFFFFFF

    def sm(v):
        v = (v + 0x9E3779B97F4A7C15) & M
        v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & M
        v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & M
        return v ^ (v >> 31)

    for i in range(2000):
        h = sm(77 ^ sm(i))
        u1 = ((h >> 40) + 1) / 2.0 ** 24
        u2 = ((h >> 16) & 0xFFFFFF) / 2.0 ** 24
        v = math.sqrt(-2 * math.log(u1)) * math.cos(2 * math.pi * u2)
        assert abs(float(z[i]) - v) <= 2 ** -23 * abs(v) + 1e-12, i


def test_generator_packing_equals_host_packer_and_gamma():
    """gen_sparse_ternary packs its latent exactly as the library's host
    packer (make_layer_from_latent) does, and its gamma (the device's double
    summation order) equals mean |W| to float rounding."""
    from spbitnet_amd import weights as Wt
    for rows, cols, seed in [(64, 256, 1), (33, 640, 2), (1, 64, 3), (300, 2560, 4)]:
        meta, values, gamma = O.gen_sparse_ternary(seed, rows, cols)
        w = O.gen_normals(seed, rows * cols).reshape(rows, cols)
        want = Wt.make_layer_from_latent(w)
        assert np.array_equal(meta, want.meta) and np.array_equal(values, want.values)
        exact = float(np.abs(w.astype(np.float64)).sum() / (rows * cols))
        assert abs(gamma - exact) <= 2 ** -23 * exact


def test_generator_bf16_embedding():
    n, std = 5000, 0.02
    got = O.gen_normal_bf16(99, n, std)
    want = O.to_bf16_bits(O.gen_normals(99, n) * np.float32(std))
    assert np.array_equal(got, want)


# ---- structured-sparse int8 GEMM (the cuSPARSELt backend) --------------------

def _prune_by_stable_argsort(A):
    """Independent statement of the pruning rule: np.argsort(|a|, kind='stable')
    ascending per group and keep the last two (python/convert_model.py:88-119's
    formulation, where the later index sorts later among equal magnitudes)."""
    m, k = A.shape
    g = A.reshape(m, k // 4, 4).astype(np.int64)
    order = np.argsort(np.abs(g), axis=-1, kind="stable")
    keep = np.zeros(g.shape, bool)
    np.put_along_axis(keep, order[..., 2:], True, axis=-1)
    return np.where(keep, g, 0).reshape(m, k).astype(np.int8)


def test_prune24_i8_brute_force_and_argsort():
    vals = np.array(list(itertools.product(range(-2, 3), repeat=4)), np.int8).reshape(1, -1)
    assert np.array_equal(O.prune24_i8(vals), _prune_by_stable_argsort(vals))
    rng = np.random.default_rng(3)
    A = rng.integers(-128, 128, (37, 256)).astype(np.int8)
    A[:, ::7] = -128  # the magnitude 128 only -128 has
    assert np.array_equal(O.prune24_i8(A), _prune_by_stable_argsort(A))
    T = rng.integers(-1, 2, (64, 256)).astype(np.int8)  # the reference test's {-1,0,1}
    assert np.array_equal(O.prune24_i8(T), _prune_by_stable_argsort(T))


def test_prune24_i8_properties():
    rng = np.random.default_rng(4)
    A = rng.integers(-128, 128, (50, 512)).astype(np.int8)
    P = O.prune24_i8(A)
    g = P.reshape(50, -1, 4)
    assert ((g != 0).sum(-1) <= 2).all()
    assert ((P == 0) | (P == A)).all()                      # kept values come from A
    assert np.array_equal(O.prune24_i8(P), P)               # idempotent
    # groups with at most two non-zeros are kept whole
    B = A.reshape(50, -1, 4).copy()
    B[..., 1] = 0
    B[..., 3] = 0
    B = B.reshape(50, 512)
    assert np.array_equal(O.prune24_i8(B), B)
    # the kept pair carries the two largest magnitudes of its group
    ga = np.abs(A.reshape(50, -1, 4).astype(np.int32))
    top2 = np.sort(ga, -1)[..., 2:].sum(-1)
    assert np.array_equal(np.abs(g.astype(np.int32)).sum(-1), top2)


def test_int8_gemm_closed_forms():
    rng = np.random.default_rng(8)
    m, k, n = 33, 260, 19
    A = rng.integers(-128, 128, (m, k)).astype(np.int8)
    B = rng.integers(-128, 128, (n, k)).astype(np.int8)
    D = O.int8_gemm(A, B)
    assert np.array_equal(D, (B.astype(np.float64) @ A.astype(np.float64).T).astype(np.int32))
    E = np.zeros((k, k), np.int8)
    np.fill_diagonal(E, 1)
    assert np.array_equal(O.int8_gemm(A, E), A.T.astype(np.int32))   # B = e_j reads column j
    ones = np.ones((1, k), np.int8)
    assert np.array_equal(O.int8_gemm(A, ones)[0], A.astype(np.int32).sum(1))
    ext = np.full((1, 4096), -128, np.int8)  # |sum| = 2^26: int32, no overflow
    assert O.int8_gemm(ext, ext)[0, 0] == 128 * 128 * 4096
