"""Pins the CPU oracle of the decode step (oracle/spb_engine_oracle.c), which
the GPU engine is required to match bit for bit, against float64
restatements of the reference's formulas (src/inference.cu:126-283,
src/kernels/inference_kernels.cu).

Each operation is checked teacher-forced: its float64 restatement is fed the
oracle's own inputs to that operation, so float32-vs-float64 differences do
not propagate.  The remaining differences are rounding-boundary flips (a bf16
rounding or an int8 quantisation landing the other way), which touch few
elements by about one bf16 ulp; a wrong formula (RoPE rotation, GQA mapping,
missing scale, sub-norm placement, relu vs relu^2, residual source, LM-head
layout) changes most elements by far more, and fails."""
import math

import numpy as np
import pytest

from forward64 import bf16, host_model, quant
from oracle import oracle as O
from spbitnet_amd import weights as W
from spbitnet_amd.model import ModelConfig


def _cfg(**kw):
    base = dict(hidden_size=256, num_hidden_layers=1, num_attention_heads=4,
                num_key_value_heads=2, intermediate_size=512, vocab_size=512,
                max_position_embeddings=256, head_dim=64, rms_norm_eps=1e-5,
                rope_theta=500000.0)
    base.update(kw)
    return ModelConfig(**base)


def _close(got, want, what, frac=0.03, ulps=2.0):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = float(np.abs(want).max()) or 1.0
    diff = np.abs(got - want)
    assert np.mean(diff > 0) <= frac, f"{what}: {np.mean(diff > 0):.3%} of elements differ"
    assert diff.max() <= ulps * 2.0 ** -7 * scale, \
        f"{what}: max |diff| {diff.max():.3g} vs scale {scale:.3g}"


def _rms64(x, w, eps):
    x = np.asarray(x, np.float64)
    return bf16(x / np.sqrt(np.mean(x * x) + eps) * w)


def _bitlinear64(x, lin, raw=False):
    """BitLinear in float64 with the int8 quantisation decisions taken from
    the oracle's own quantiser (pinned in test_oracle.py); every position
    where they differ from float64 rounding must sit on a rounding boundary."""
    meta, values, gamma, rows, cols, _, _ = lin
    dense = W.unpack(meta, values, rows, cols).astype(np.float64)
    x64 = np.asarray(x, np.float64)
    q64, a = quant(x64)
    q32, a32 = O.quantize(np.asarray(x, np.float32))
    assert a32 == a
    off = np.flatnonzero(q64 != q32)
    assert len(off) <= max(4, x64.size // 50)
    t = x64[off] * (127.0 / a)
    assert np.all(np.abs(np.abs(t - np.floor(t)) - 0.5) < 1e-4), "quantisation differs off a boundary"
    y = (dense @ q32.astype(np.float64)) * (gamma * a / 127.0)
    return y if raw else bf16(y)


def _rope64(v, pos, cfg):
    hd = cfg.head_dim
    i = np.arange(hd // 2)
    freq = 1.0 / np.power(float(np.float32(cfg.rope_theta)), 2.0 * i / hd)
    ang = pos * freq
    v = np.asarray(v, np.float64).reshape(-1, hd // 2, 2)
    x0, x1 = v[..., 0], v[..., 1]
    return bf16(np.stack([x0 * np.cos(ang) - x1 * np.sin(ang),
                          x0 * np.sin(ang) + x1 * np.cos(ang)], -1).reshape(-1))


@pytest.mark.parametrize("nkv,sub_norms,max_seq,n_pos", [
    (2, True, 128, 70), (4, True, 128, 70), (1, False, 128, 70),
    (2, True, 512, 300)])  # five 64-position splits
def test_engine_oracle_teacher_forced(nkv, sub_norms, max_seq, n_pos):
    cfg = _cfg(num_key_value_heads=nkv)
    H, I, hd, nh = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim, cfg.num_attention_heads
    kvd = nkv * hd
    host = host_model(cfg, seed=nkv, qk_gamma=0.02, sub_norms=sub_norms, norm_jitter=0.1)
    L = host["layers"][0]
    n_in, n_post, n_sub, n_ffn = L["norms"]
    e = O.EngineOracle(host, max_seq)
    emb = (np.asarray(host["embed"], np.uint32) << 16).view(np.float32).astype(np.float64)
    ks, vs = [], []
    toks = [int(t) for t in np.random.default_rng(nkv).integers(0, cfg.vocab_size, n_pos)]
    for pos, tok in enumerate(toks):
        argmax, logits = e.step(tok)
        x_in = emb[tok]
        h = e.debug("h")
        _close(h, _rms64(x_in, n_in, cfg.rms_norm_eps), f"input norm @{pos}")
        qkv = e.debug("qkv")
        want = np.concatenate([_bitlinear64(h, L[p]) for p in ("q_proj", "k_proj", "v_proj")])
        _close(qkv, want, f"qkv @{pos}")
        # attention from the oracle's own q/k/v, float64 softmax (inference_kernels.cu:241-371)
        q = _rope64(qkv[:H], pos, cfg).reshape(nh, hd)
        ks.append(_rope64(qkv[H:H + kvd], pos, cfg).reshape(nkv, hd))
        vs.append(np.asarray(qkv[H + kvd:], np.float64).reshape(nkv, hd))
        K, V = np.stack(ks, 1), np.stack(vs, 1)  # [nkv][pos+1][hd]
        att = np.empty(H)
        for hh in range(nh):
            kv = hh * nkv // nh
            s = K[kv] @ q[hh] / math.sqrt(hd)
            p = np.exp(s - s.max())
            att[hh * hd:(hh + 1) * hd] = (p / p.sum()) @ V[kv]
        attn = e.debug("attn")
        _close(attn, bf16(att), f"attention @{pos}")
        o = e.debug("o")
        o_want = _bitlinear64(attn, L["o_proj"])
        if n_sub is not None:
            o_want = _rms64(o_want, n_sub, cfg.rms_norm_eps)
        _close(o, o_want, f"o_proj + sub-norm @{pos}")
        x_mid = e.debug("x_mid")
        _close(x_mid, bf16(np.asarray(o, np.float64) + x_in), f"attention residual @{pos}", frac=0.0)
        h2 = _rms64(x_mid, n_post, cfg.rms_norm_eps)
        gu = e.debug("gate_up")
        _close(gu, np.concatenate([_bitlinear64(h2, L["gate_proj"]),
                                   _bitlinear64(h2, L["up_proj"])]), f"gate/up @{pos}")
        g, u = np.asarray(gu[:I], np.float64), np.asarray(gu[I:], np.float64)
        mm = np.maximum(g, 0.0) ** 2 * u
        m = e.debug("m")
        _close(m, _rms64(mm, n_ffn, cfg.rms_norm_eps) if n_ffn is not None else bf16(mm),
               f"relu2 + ffn sub-norm @{pos}")
        x_out = e.hidden()
        _close(x_out, bf16(bf16(_bitlinear64(m, L["down_proj"], raw=True)) + x_mid),
               f"down + residual @{pos}")
        xn = e.debug("xn")
        _close(xn, _rms64(x_out, host["final_norm"], cfg.rms_norm_eps), f"final norm @{pos}")
        lg = emb @ np.asarray(xn, np.float64)
        assert np.abs(logits - lg).max() <= 1e-5 * np.abs(lg).max() + 1e-6, f"logits @{pos}"
        top2 = np.sort(lg)[-2:]
        if top2[1] - top2[0] > 1e-4 * np.abs(lg).max():
            assert argmax == int(np.argmax(lg))


def test_engine_oracle_catches_planted_mistakes():
    """The checks above fail on a plausible mistake: here a RoPE with the
    rotation reversed and a GQA mapping by modulo, planted in the float64
    side (the oracle is unchanged)."""
    cfg = _cfg(num_key_value_heads=2)
    H, hd, nh, nkv = cfg.hidden_size, cfg.head_dim, cfg.num_attention_heads, 2
    kvd = nkv * hd
    host = host_model(cfg, seed=5, qk_gamma=0.02)
    e = O.EngineOracle(host, 64)
    toks = [3, 17, 99, 250, 7]
    ks, vs = [], []
    for pos, tok in enumerate(toks):
        e.step(tok)
        qkv = e.debug("qkv")
        q = _rope64(qkv[:H], -pos, cfg).reshape(nh, hd)  # wrong direction
        ks.append(_rope64(qkv[H:H + kvd], -pos, cfg).reshape(nkv, hd))
        vs.append(np.asarray(qkv[H + kvd:], np.float64).reshape(nkv, hd))
    K, V = np.stack(ks, 1), np.stack(vs, 1)
    att = np.empty(H)
    for hh in range(nh):
        kv = hh % nkv  # wrong mapping (reference: hh * nkv // nh)
        s = K[kv] @ q[hh] / math.sqrt(hd)
        p = np.exp(s - s.max())
        att[hh * hd:(hh + 1) * hd] = (p / p.sum()) @ V[kv]
    with pytest.raises(AssertionError):
        _close(e.debug("attn"), bf16(att), "planted")


def test_exp_neg_accuracy():
    xs = np.concatenate([-np.logspace(-8, np.log10(86.0), 4000), [0.0, -1e-30, -85.99]]).astype(np.float32)
    for x in xs:
        got = O.exp_neg(float(x))
        want = math.exp(float(x))
        assert abs(got - want) <= 3 * np.spacing(np.float32(want)), (x, got, want)
    assert O.exp_neg(0.0) == 1.0
    assert O.exp_neg(-86.5) == 0.0 and O.exp_neg(-1000.0) == 0.0


def test_engine_oracle_refuses_full_cache():
    cfg = _cfg()
    e = O.EngineOracle(host_model(cfg, seed=1), 3)
    for t in (1, 2, 3):
        e.step(t)
    with pytest.raises(ValueError):
        e.step(4)
    e.reset()
    with pytest.raises(ValueError):
        e.step(cfg.vocab_size)

