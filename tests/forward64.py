"""Float64 restatement of the reference decode step (src/inference.cu:126-283,
src/kernels/inference_kernels.cu) in numpy, used to pin the CPU oracle's
engine step: textbook formulas evaluated in float64 with the reference's
storage roundings (16-bit activations, here bf16; int8 absmax quantisation;
exact int32 GEMV), probabilities normalised before the V sum as in
softmax_kernel + attention_output_kernel, rsqrt and exp in float64.
"""
from __future__ import annotations

import numpy as np

from spbitnet_amd import weights as W


def bf16(x):
    """Round float64/float32 values to bf16 (through float32, RNE), as float64."""
    f = np.asarray(x, np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def quant(x):
    """absmax int8 quantisation (inference_kernels.cu:69-114)."""
    a = float(np.max(np.abs(x))) if x.size else 0.0
    s = 127.0 / a if a > 0 else 0.0
    return np.clip(np.rint(x * s), -128, 127), a


class Forward64:
    PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

    def __init__(self, host: dict, max_seq: int):
        self.c = c = host["config"]
        self.max_seq = max_seq
        self.layers = []
        for d in host["layers"]:
            L = {}
            for p in self.PROJ:
                m, v, g, rows, cols, _, _ = d[p]
                L[p] = (W.unpack(m, v, rows, cols).astype(np.float64), float(g))
            L["norms"] = [None if t is None else np.asarray(t, np.float64) for t in d["norms"]]
            self.layers.append(L)
        to64 = lambda b: (np.asarray(b, np.uint32) << 16).view(np.float32).astype(np.float64)
        self.embed = to64(host["embed"])
        self.lm = self.embed if host["lm_head"] is None else to64(host["lm_head"])
        self.final_norm = np.asarray(host["final_norm"], np.float64)
        hd, nkv = c.head_dim, c.num_key_value_heads
        self.kc = [np.zeros((nkv, max_seq, hd)) for _ in self.layers]
        self.vc = [np.zeros((nkv, max_seq, hd)) for _ in self.layers]
        self.pos = 0

    def rms(self, x, w):
        return bf16(x / np.sqrt(np.mean(x * x) + self.c.rms_norm_eps) * w)

    def bitlinear(self, x, lin):
        dense, gamma = lin
        q, a = quant(x)
        return bf16((dense @ q) * (gamma * a / 127.0))

    def rope(self, v, heads):
        c = self.c
        hd = c.head_dim
        i = np.arange(hd // 2)
        freq = 1.0 / np.power(float(c.rope_theta), 2.0 * i / hd)
        ang = self.pos * freq
        cs, sn = np.cos(ang), np.sin(ang)
        v = v.reshape(heads, hd // 2, 2)
        x0, x1 = v[..., 0], v[..., 1]
        return bf16(np.stack([x0 * cs - x1 * sn, x0 * sn + x1 * cs], -1).reshape(-1))

    def step(self, token: int):
        c = self.c
        H, hd, nh, nkv = c.hidden_size, c.head_dim, c.num_attention_heads, c.num_key_value_heads
        x = self.embed[token].copy()
        for li, L in enumerate(self.layers):
            r = x
            h = self.rms(r, L["norms"][0])
            q = self.rope(self.bitlinear(h, L["q_proj"]), nh)
            k = self.rope(self.bitlinear(h, L["k_proj"]), nkv)
            v = self.bitlinear(h, L["v_proj"])
            self.kc[li][:, self.pos] = k.reshape(nkv, hd)
            self.vc[li][:, self.pos] = v.reshape(nkv, hd)
            n = self.pos + 1
            att = np.empty(H)
            for hh in range(nh):
                kv = hh * nkv // nh
                s = self.kc[li][kv, :n] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                att[hh * hd:(hh + 1) * hd] = p @ self.vc[li][kv, :n]
            att = bf16(att)
            o = self.bitlinear(att, L["o_proj"])
            if L["norms"][2] is not None:
                o = self.rms(o, L["norms"][2])
            x = bf16(o + r)
            r = x
            h = self.rms(x, L["norms"][1])
            g = self.bitlinear(h, L["gate_proj"])
            u = self.bitlinear(h, L["up_proj"])
            m = np.maximum(g, 0.0) ** 2 * u
            m = self.rms(m, L["norms"][3]) if L["norms"][3] is not None else bf16(m)
            d = self.bitlinear(m, L["down_proj"])
            x = bf16(d + r)
        xn = self.rms(x, self.final_norm)
        self.pos += 1
        return self.lm @ xn


def host_model(cfg, seed=0, qk_gamma=None, sub_norms=True, norm_jitter=0.0):
    """A random model as host arrays in the layout Model.to_host() returns,
    generated on the CPU (spbitnet_amd.weights) for the CPU-only checks.
    qk_gamma overrides the q/k projection gamma (a well-conditioned softmax);
    norm_jitter draws RMSNorm weights from 1 + jitter * N(0,1)."""
    from oracle import oracle as O
    H, I = cfg.hidden_size, cfg.intermediate_size
    kvd = cfg.num_key_value_heads * cfg.head_dim
    shapes = {"q_proj": (H, H), "k_proj": (kvd, H), "v_proj": (kvd, H), "o_proj": (H, H),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}

    def norm(n, *tag):
        if not norm_jitter:
            return np.ones(n, np.float32)
        return (1.0 + norm_jitter * W.normal_f32(W.seed_for("norm", seed, *tag), n)).astype(np.float32)

    layers = []
    for l in range(cfg.num_hidden_layers):
        d = {}
        for p, (r, k) in shapes.items():
            L = W.random_layer(r, k, W.seed_for("host", seed, l, p))
            g = L.gamma if (qk_gamma is None or p not in ("q_proj", "k_proj")) else qk_gamma
            d[p] = (L.meta, L.values, g, r, k, L.meta.shape[1], L.values.shape[1])
        d["norms"] = [norm(H, l, 0), norm(H, l, 1),
                      norm(H, l, 2) if sub_norms else None, norm(I, l, 3) if sub_norms else None]
        layers.append(d)
    emb = (W.normal_f32(W.seed_for("host", seed, "embed"), cfg.vocab_size * H) * 0.02)
    return {"config": cfg, "layers": layers,
            "embed": O.to_bf16_bits(emb.astype(np.float32)).reshape(cfg.vocab_size, H),
            "lm_head": None, "final_norm": norm(H, "final")}
