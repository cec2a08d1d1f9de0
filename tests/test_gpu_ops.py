"""GPU checks of the per-op inference kernels (spb_rms_norm_*, spb_rope_*, ...,
the reference's include/spbitnet/inference_kernels.h wrappers) against float64
restatements of the reference formulas (src/kernels/inference_kernels.cu).

Tolerances: results stored in 16 bits may differ from the float64 value
rounded to that type by one unit in the last place (the kernels round a
float32 result once); float32 outputs are held to 1e-4 relative (5e-6 for
softmax).  Elementwise ops with a fixed float32 expression (relu2 * up,
residual add, conversion) are bit-exact against numpy float32."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

KINDS = {"f16": torch.float16, "bf16": torch.bfloat16}


def _lib():
    from spbitnet_amd import _lib as L
    return L.load(), L


def _call(name, *args):
    lib, L = _lib()
    rc = getattr(lib, name)(*args)
    L.check(rc, name)


def _p(t):
    return t.data_ptr()


def _to_host(t):
    return t.float().cpu().numpy().astype(np.float64)


def _round16(x, kind):
    x = np.asarray(x, np.float64)
    if kind == "f16":
        return x.astype(np.float32).astype(np.float16).astype(np.float64)
    return O.bf16_bits_to_f32(O.to_bf16_bits(x.astype(np.float32))).astype(np.float64)


def _ulp16(x, kind):
    x = np.abs(np.asarray(x, np.float64))
    if kind == "f16":
        return np.maximum(np.spacing(x.astype(np.float16)).astype(np.float64), 2.0 ** -24)
    e = np.floor(np.log2(np.maximum(x, 1e-38)))
    return 2.0 ** (e - 7)


def _assert_16(got, want, kind, what):
    r = _round16(want, kind)
    err = np.abs(got - r)
    bad = err > _ulp16(r, kind) * 1.01
    assert not bad.any(), f"{what}: {bad.sum()} elements off by more than 1 ulp, max {err.max()}"


def _rand16(n, kind, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * scale).to(KINDS[kind]).cuda()


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("n", [1, 7, 2560, 6912, 10000])
def test_rms_norm(gpu, kind, n):
    x = _rand16(n, kind, 3.0, n)
    w = (torch.rand(n, generator=torch.Generator().manual_seed(1)) + 0.5).cuda()
    y = torch.empty_like(x)
    _call(f"spb_rms_norm_{kind}", _p(x), _p(w), _p(y), n, 1e-5, None)
    xs = _to_host(x)
    want = xs / np.sqrt(np.mean(xs * xs) + 1e-5) * w.double().cpu().numpy()
    _assert_16(_to_host(y), want, kind, "rms_norm")
    # in place (the reference normalises d_q_ in place, src/inference.cu:207)
    _call(f"spb_rms_norm_{kind}", _p(x), _p(w), _p(x), n, 1e-5, None)
    assert torch.equal(x, y)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_rms_norm_f32in(gpu, kind):
    n = 6912
    x = (torch.randn(n, generator=torch.Generator().manual_seed(3)) * 1e4).cuda()
    w = torch.ones(n).cuda()
    y = torch.empty(n, dtype=KINDS[kind], device="cuda")
    _call(f"spb_rms_norm_f32in_{kind}", _p(x), _p(w), _p(y), n, 1e-5, None)
    xs = x.double().cpu().numpy()
    _assert_16(_to_host(y), xs / np.sqrt(np.mean(xs * xs) + 1e-5), kind, "rms_norm_f32in")


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("nh,hd,pos", [(20, 128, 0), (20, 128, 1234), (5, 64, 4095), (3, 2, 7)])
def test_rope(gpu, kind, nh, hd, pos):
    v = _rand16(nh * hd, kind, 2.0, pos)
    x = _to_host(v).reshape(nh, hd // 2, 2)
    _call(f"spb_rope_{kind}", _p(v), nh, hd, pos, 500000.0, None)
    i = np.arange(hd // 2)
    ang = pos * (1.0 / np.power(500000.0, 2.0 * i / hd))
    want = np.stack([x[..., 0] * np.cos(ang) - x[..., 1] * np.sin(ang),
                     x[..., 0] * np.sin(ang) + x[..., 1] * np.cos(ang)], -1).reshape(-1)
    # angle is a float32 product (inference_kernels.cu:197): allow its rounding
    got = _to_host(v)
    tol = _ulp16(_round16(want, kind), kind) * 1.01 + 1e-6 * pos * np.abs(x).max()
    assert np.all(np.abs(got - _round16(want, kind)) <= tol)


def test_scatter_kv(gpu):
    nkv, hd, max_seq = 5, 128, 64
    cache = torch.zeros(nkv * max_seq * hd, dtype=torch.bfloat16, device="cuda")
    src = _rand16(nkv * hd, "bf16", 1.0, 9)
    _call("spb_scatter_kv", _p(src), _p(cache), nkv, hd, max_seq, 37, None)
    c = cache.view(nkv, max_seq, hd)
    assert torch.equal(c[:, 37], src.view(nkv, hd))
    assert int((c != 0).sum()) == int((src != 0).sum())
    lib, L = _lib()
    with pytest.raises(L.SpbError):
        _call("spb_scatter_kv", _p(src), _p(cache), nkv, hd, max_seq, max_seq, None)


def test_scatter_kv_reference_kat(gpu):
    """The reference's ScatterKV case (tests/test_inference_kernels.cu:459-491):
    two kv heads of 4 values [1..4] and [5..8] into an 8-position cache at
    position 3; those land at [head][3][:], everything else stays zero."""
    nkv, hd, max_seq, pos = 2, 4, 8, 3
    src = torch.tensor([1, 2, 3, 4, 5, 6, 7, 8], dtype=torch.float16, device="cuda")
    cache = torch.zeros(nkv * max_seq * hd, dtype=torch.float16, device="cuda")
    _call("spb_scatter_kv", _p(src), _p(cache), nkv, hd, max_seq, pos, None)
    want = np.zeros((nkv, max_seq, hd))
    want[0, pos] = [1, 2, 3, 4]
    want[1, pos] = [5, 6, 7, 8]
    assert np.array_equal(cache.view(nkv, max_seq, hd).float().cpu().numpy(), want)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_attention_single_head_reference_kat(gpu, kind):
    """The reference's AttentionSingleHead case (tests/test_inference_kernels.cu:376-453):
    q = [1,0,1,0] against K rows [1,0,0,0], [0,1,0,1], [1,0,1,0] scores
    0.5, 0 and 1.0 (dot products 1, 0, 2 times 1/sqrt(4)); the softmax of
    those sums to 1 with score 2 largest and score 1 smallest; the output is
    the weights times V rows [10,0,0,0], [0,20,0,0], [0,0,30,0].  Held here to
    the kernels' own tolerances (float32 scores exact for these inputs,
    softmax within 5e-6, output within one 16-bit ulp) rather than the
    reference test's 1e-3 / 1e-4 / 0.1."""
    nh, nkv, hd, max_seq, seq = 1, 1, 4, 8, 3
    dt = KINDS[kind]
    q = torch.tensor([1, 0, 1, 0], dtype=dt, device="cuda")
    K = torch.zeros(max_seq, hd, dtype=dt)
    K[0, 0] = 1
    K[1, 1] = 1
    K[1, 3] = 1
    K[2, 0] = 1
    K[2, 2] = 1
    V = torch.zeros(max_seq, hd, dtype=dt)
    V[0, 0], V[1, 1], V[2, 2] = 10, 20, 30
    K, V = K.cuda(), V.cuda()
    sc = torch.zeros(nh * max_seq, dtype=torch.float32, device="cuda")
    _call(f"spb_attention_scores_{kind}", _p(q), _p(K), _p(sc), nh, nkv, hd, max_seq, seq,
          0.5, None)
    assert sc[:3].cpu().tolist() == [0.5, 0.0, 1.0]
    assert torch.all(sc[3:] == 0)
    _call("spb_softmax", _p(sc), nh, max_seq, seq, None)
    p = sc[:3].double().cpu().numpy()
    e = np.exp(np.array([0.5, 0.0, 1.0]) - 1.0)
    assert np.allclose(p, e / e.sum(), rtol=5e-6, atol=0)
    assert abs(p.sum() - 1.0) < 1e-6 and p[2] > p[0] > p[1]
    out = torch.empty(nh * hd, dtype=dt, device="cuda")
    _call(f"spb_attention_output_{kind}", _p(sc), _p(V), _p(out), nh, nkv, hd, max_seq, seq, None)
    want = np.array([10 * p[0], 20 * p[1], 30 * p[2], 0.0])
    got = _to_host(out)
    assert np.all(np.abs(got - _round16(want, kind)) <= _ulp16(_round16(want, kind), kind) * 1.01)
    assert got[3] == 0.0


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("nh,nkv,hd,seq", [(20, 5, 128, 1), (20, 5, 128, 333), (8, 8, 64, 70),
                                           (4, 1, 256, 17)])
def test_attention_scores_softmax_output(gpu, kind, nh, nkv, hd, seq):
    max_seq = 512
    q = _rand16(nh * hd, kind, 1.0, 1)
    K = _rand16(nkv * max_seq * hd, kind, 1.0, 2)
    V = _rand16(nkv * max_seq * hd, kind, 1.0, 3)
    sc = torch.zeros(nh * max_seq, dtype=torch.float32, device="cuda")
    scale = 1.0 / np.sqrt(hd)
    _call(f"spb_attention_scores_{kind}", _p(q), _p(K), _p(sc), nh, nkv, hd, max_seq, seq,
          float(scale), None)
    qh, Kh, Vh = _to_host(q).reshape(nh, hd), _to_host(K).reshape(nkv, max_seq, hd), \
        _to_host(V).reshape(nkv, max_seq, hd)
    kv = np.arange(nh) * nkv // nh
    s64 = np.einsum("hd,hjd->hj", qh, Kh[kv, :seq]) * np.float32(scale)
    got = sc.view(nh, max_seq)[:, :seq].double().cpu().numpy()
    assert np.allclose(got, s64, rtol=1e-4, atol=1e-4 * np.abs(s64).max())
    assert torch.all(sc.view(nh, max_seq)[:, seq:] == 0)
    _call("spb_softmax", _p(sc), nh, max_seq, seq, None)
    p64 = np.exp(got - got.max(1, keepdims=True))
    p64 /= p64.sum(1, keepdims=True)
    pg = sc.view(nh, max_seq)[:, :seq].double().cpu().numpy()
    assert np.allclose(pg, p64, rtol=5e-6, atol=1e-7)
    out = torch.empty(nh * hd, dtype=KINDS[kind], device="cuda")
    _call(f"spb_attention_output_{kind}", _p(sc), _p(V), _p(out), nh, nkv, hd, max_seq, seq, None)
    want = np.einsum("hj,hjd->hd", pg, Vh[kv, :seq]).reshape(-1)
    got_o = _to_host(out)
    err = np.abs(got_o - _round16(want, kind))
    assert np.all(err <= _ulp16(_round16(want, kind), kind) * 1.01 + 1e-6)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_elementwise_bit_exact(gpu, kind):
    n = 6912 + 5
    g, u = _rand16(n, kind, 4.0, 1), _rand16(n, kind, 4.0, 2)
    gf, uf = g.float().cpu().numpy(), u.float().cpu().numpy()
    r = np.maximum(np.float32(0), gf)
    want32 = (r * r) * uf                                  # float32, as relu2_mul_f32_kernel
    o32 = torch.empty(n, dtype=torch.float32, device="cuda")
    _call(f"spb_relu2_mul_f32_{kind}", _p(g), _p(u), _p(o32), n, None)
    assert np.array_equal(o32.cpu().numpy(), want32)
    o16 = torch.empty(n, dtype=KINDS[kind], device="cuda")
    _call(f"spb_relu2_mul_{kind}", _p(g), _p(u), _p(o16), n, None)
    assert np.array_equal(o16.float().cpu().numpy(), _round16(want32, kind).astype(np.float32))
    c16 = torch.empty(n, dtype=KINDS[kind], device="cuda")
    _call(f"spb_float_to_{kind}", _p(o32), _p(c16), n, None)
    assert torch.equal(c16, o16)
    a = torch.empty(n, dtype=KINDS[kind], device="cuda")
    _call(f"spb_residual_add_{kind}", _p(g), _p(u), _p(a), n, None)
    assert np.array_equal(a.float().cpu().numpy(), _round16(gf + uf, kind).astype(np.float32))


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("rows,cols", [(1000, 2560), (77, 1003), (128256 // 64, 2560)])
def test_gemv16(gpu, kind, rows, cols):
    W = _rand16(rows * cols, kind, 0.05, rows)
    x = _rand16(cols, kind, 1.0, cols)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    _call(f"spb_gemv_{kind}", _p(W), _p(x), _p(y), rows, cols, None)
    want = _to_host(W).reshape(rows, cols) @ _to_host(x)
    got = y.double().cpu().numpy()
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())


def test_argmax_lowest_index_on_ties(gpu):
    x = torch.randn(128256, generator=torch.Generator().manual_seed(5)).cuda()
    x[1000] = 7.0
    x[90000] = 7.0
    x[5] = float("nan")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    _call("spb_argmax_f32", _p(x), x.numel(), _p(out), None)
    assert int(out.item()) == 1000
    y = torch.full((3,), -1.0, device="cuda")
    _call("spb_argmax_f32", _p(y), 3, _p(out), None)
    assert int(out.item()) == 0
