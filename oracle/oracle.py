"""numpy-level access to the CPU checker (oracle/spb_oracle.c) and, when built,
to the reference's own format code (oracle/_ref/libspb_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the spbitnet_amd package.  Each wrapper
names the reference file:line its C function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libspb_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libspb_ref.so")

_lib = None
_ref = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


def build() -> None:
    """Compile the checker (and the reference-header bridge where the
    reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = ctypes.CDLL(ORACLE_SO)
        L.spbo_meta_stride.argtypes = [_I]
        L.spbo_values_stride.argtypes = [_I]
        L.spbo_mask_top2.argtypes = [_P, _I, _I, _P]
        L.spbo_kept_sign.argtypes = [_P, _P, _I, _P]
        L.spbo_absmean.argtypes = [_P, ctypes.c_size_t]
        L.spbo_absmean.restype = ctypes.c_double
        L.spbo_pack.argtypes = [_P, _P, _I, _I, _P, _P]
        L.spbo_unpack.argtypes = [_P, _P, _I, _I, _I, _I, _P]
        L.spbo_gemv.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I]
        L.spbo_gemm.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I]
        L.spbo_dense_mac.argtypes = [_P, _P, _P, _I, _I]
        L.spbo_absmax.argtypes = [_P, _I]
        L.spbo_absmax.restype = _F
        L.spbo_quant_scale.argtypes = [_F]
        L.spbo_quant_scale.restype = _F
        L.spbo_round_clamp.argtypes = [_F]
        L.spbo_quantize.argtypes = [_P, _I, _P]
        L.spbo_quantize.restype = _F
        L.spbo_dequant_scale.argtypes = [_F, _F]
        L.spbo_dequant_scale.restype = _F
        L.spbo_dequant.argtypes = [_P, _I, _F, _F, _P]
        L.spbo_fused_bitlinear.argtypes = [_P, _P, _P, _F, _F, _I, _I, _I, _I, _P, _P]
        L.spbo_bf16_round_array.argtypes = [_P, _I, _P]
        L.spbo_planes.argtypes = [_P, _I, _P]
        L.spbo_prune24_i8.argtypes = [_P, _I, _I, _P]
        L.spbo_int8_gemm.argtypes = [_P, _P, _P, _I, _I, _I]
        L.spbo_gen_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.spbo_gen_normal.restype = _F
        L.spbo_gen_ln_u24.argtypes = [ctypes.c_uint32]
        L.spbo_gen_ln_u24.restype = ctypes.c_double
        L.spbo_gen_sqrt.argtypes = [ctypes.c_double]
        L.spbo_gen_sqrt.restype = ctypes.c_double
        L.spbo_gen_cos_u24.argtypes = [ctypes.c_uint32]
        L.spbo_gen_cos_u24.restype = ctypes.c_double
        L.spbo_gen_normals.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_long, _P]
        L.spbo_gen_normal_bf16.argtypes = [ctypes.c_uint64, ctypes.c_long, _F, _P]
        L.spbo_gen_gamma.argtypes = [_P, _I, _I]
        L.spbo_gen_gamma.restype = _F
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref():
    """The reference's own SparseTernaryTensor code, via oracle/ref_bridge.cpp."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(REF_SO)
        R.ref_meta_stride.argtypes = [_I]
        R.ref_values_stride.argtypes = [_I]
        R.ref_pack_from_dense.argtypes = [_P, _P, _I, _I, _P, _P]
        R.ref_pack_with_pruning.argtypes = [_P, _I, _I, _P, _P]
        R.ref_unpack.argtypes = [_P, _P, _I, _I, _P]
        R.ref_make_test_case.argtypes = [ctypes.c_uint, _I, _I, _I, _P, _P, _P]
        R.ref_cpu_sparse_gemv.argtypes = [_P, _P, _P, _P, _I, _I]
        _ref = R
    return _ref


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def meta_stride(cols: int) -> int:
    """sparse_ternary_tensor.h:254-257"""
    return lib().spbo_meta_stride(cols)


def values_stride(cols: int) -> int:
    """sparse_ternary_tensor.h:261-264"""
    return lib().spbo_values_stride(cols)


def mask_top2(w: np.ndarray) -> np.ndarray:
    """python/convert_model.py:88-119 (stable argsort: higher index wins ties)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    m = np.zeros((rows, cols), np.uint8)
    lib().spbo_mask_top2(_p(w), rows, cols, _p(m))
    return m


def kept_sign(w: np.ndarray, mask: np.ndarray) -> np.ndarray:
    """python/convert_model.py:270-283 (kept value = sign(w), w >= 0 -> +1)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    mask = np.ascontiguousarray(mask, dtype=np.uint8)
    out = np.zeros(w.shape, np.int8)
    lib().spbo_kept_sign(_p(w), _p(mask), w.size, _p(out))
    return out


def absmean(w: np.ndarray) -> float:
    """python/convert_model.py:132 (in double; see spb_oracle.c)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    return lib().spbo_absmean(_p(w), w.size)


def pack(w: np.ndarray, mask: np.ndarray):
    """SparseTernaryTensor::pack_from_dense (sparse_ternary_tensor.h:58-108)."""
    w = np.ascontiguousarray(w, dtype=np.int8)
    mask = np.ascontiguousarray(mask, dtype=np.uint8)
    rows, cols = w.shape
    meta = np.zeros((rows, meta_stride(cols)), np.uint32)
    values = np.zeros((rows, values_stride(cols)), np.uint32)
    rc = lib().spbo_pack(_p(w), _p(mask), rows, cols, _p(meta), _p(values))
    if rc != 0:
        raise ValueError(f"spbo_pack failed ({rc}): cols%4 or a group without exactly 2 kept")
    return meta, values


def unpack(meta: np.ndarray, values: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """SparseTernaryTensor::unpack_to_int8 (sparse_ternary_tensor.h:197-232)."""
    meta = np.ascontiguousarray(meta, dtype=np.uint32)
    values = np.ascontiguousarray(values, dtype=np.uint32)
    out = np.zeros((rows, cols), np.int8)
    lib().spbo_unpack(_p(meta), _p(values), rows, cols, meta.shape[-1], values.shape[-1], _p(out))
    return out


def gemv(meta, values, x, rows, cols) -> np.ndarray:
    """cpu_sparse_gemv (tests/test_sparse_ternary.cu:17-33)."""
    meta = np.ascontiguousarray(meta, dtype=np.uint32)
    values = np.ascontiguousarray(values, dtype=np.uint32)
    x = np.ascontiguousarray(x, dtype=np.int8)
    y = np.zeros(rows, np.int32)
    lib().spbo_gemv(_p(meta), _p(values), _p(x), _p(y), rows, cols, meta.shape[-1], values.shape[-1])
    return y


def dense_mac(dense: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y = dense @ x in int32 (the MAC of cpu_sparse_gemv without its unpack)."""
    dense = np.ascontiguousarray(dense, dtype=np.int8)
    x = np.ascontiguousarray(x, dtype=np.int8)
    rows, cols = dense.shape
    y = np.zeros(rows, np.int32)
    lib().spbo_dense_mac(_p(dense), _p(x), _p(y), rows, cols)
    return y


def gemm(meta, values, X, rows, cols) -> np.ndarray:
    """cpu_int8_gemm (tests/test_cusparselt.cu:16-28), token-major X[n][cols] -> Y[n][rows]."""
    meta = np.ascontiguousarray(meta, dtype=np.uint32)
    values = np.ascontiguousarray(values, dtype=np.uint32)
    X = np.ascontiguousarray(X, dtype=np.int8)
    n = X.shape[0]
    Y = np.zeros((n, rows), np.int32)
    lib().spbo_gemm(_p(meta), _p(values), _p(X), _p(Y), rows, cols, n, meta.shape[-1], values.shape[-1])
    return Y


def absmax(x: np.ndarray) -> float:
    """absmax_reduce_kernel (src/kernels/inference_kernels.cu:120-148)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(np.float32(lib().spbo_absmax(_p(x), x.size)))


def quantize(x: np.ndarray):
    """absmax_quantize_kernel (src/kernels/inference_kernels.cu:69-114) -> (q, absmax)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.size, np.int8)
    a = lib().spbo_quantize(_p(x), x.size, _p(q))
    return q, float(np.float32(a))


def dequant(acc: np.ndarray, gamma: float, absmax_: float) -> np.ndarray:
    """dequantize_kernel (src/kernels/inference_kernels.cu:162-171), float32 before the final cast."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    out = np.zeros(acc.size, np.float32)
    lib().spbo_dequant(_p(acc), acc.size, float(gamma), float(absmax_), _p(out))
    return out


def fused_bitlinear(meta, values, x_f32, absmax_, gamma, rows, cols):
    """fused_sparse_bitlinear_kernel (src/kernels/sparse_ternary.cu:181-234).
    Returns (float32 output before the 16-bit cast, int32 accumulators)."""
    meta = np.ascontiguousarray(meta, dtype=np.uint32)
    values = np.ascontiguousarray(values, dtype=np.uint32)
    x = np.ascontiguousarray(x_f32, dtype=np.float32)
    out = np.zeros(rows, np.float32)
    acc = np.zeros(rows, np.int32)
    lib().spbo_fused_bitlinear(_p(meta), _p(values), _p(x), float(absmax_), float(gamma), rows, cols,
                               meta.shape[-1], values.shape[-1], _p(out), _p(acc))
    return out, acc


def planes(x: np.ndarray) -> np.ndarray:
    """Bit-plane activation layout: word [w*8+b] bit j = bit b of x[32w+j]."""
    x = np.ascontiguousarray(x, dtype=np.int8)
    out = np.zeros(8 * ((x.size + 31) // 32), np.uint32)
    lib().spbo_planes(_p(x), x.size, _p(out))
    return out


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size, np.uint16)
    lib().spbo_bf16_round_array(_p(x), x.size, _p(out))
    return out.reshape(x.shape)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> fp16 bit patterns, round to nearest even (IEEE, as __float2half)."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


# ---- reference's own code (oracle/_ref), where built ------------------------

def ref_pack_from_dense(w, mask):
    w = np.ascontiguousarray(w, dtype=np.int8)
    mask = np.ascontiguousarray(mask, dtype=np.uint8)
    rows, cols = w.shape
    R = ref()
    meta = np.zeros((rows, R.ref_meta_stride(cols)), np.uint32)
    values = np.zeros((rows, R.ref_values_stride(cols)), np.uint32)
    R.ref_pack_from_dense(_p(w), _p(mask), rows, cols, _p(meta), _p(values))
    return meta, values


def ref_pack_with_pruning(latent):
    latent = np.ascontiguousarray(latent, dtype=np.float32)
    rows, cols = latent.shape
    R = ref()
    meta = np.zeros((rows, R.ref_meta_stride(cols)), np.uint32)
    values = np.zeros((rows, R.ref_values_stride(cols)), np.uint32)
    R.ref_pack_with_pruning(_p(latent), rows, cols, _p(meta), _p(values))
    return meta, values


def ref_unpack(meta, values, rows, cols):
    meta = np.ascontiguousarray(meta, dtype=np.uint32)
    values = np.ascontiguousarray(values, dtype=np.uint32)
    out = np.zeros((rows, cols), np.int8)
    ref().ref_unpack(_p(meta), _p(values), rows, cols, _p(out))
    return out


def ref_cpu_sparse_gemv(meta, values, x, rows, cols):
    """The reference's CPU GEMV: its own unpack_to_int8 + dense int32 MAC."""
    meta = np.ascontiguousarray(meta, dtype=np.uint32)
    values = np.ascontiguousarray(values, dtype=np.uint32)
    x = np.ascontiguousarray(x, dtype=np.int8)
    y = np.zeros(rows, np.int32)
    ref().ref_cpu_sparse_gemv(_p(meta), _p(values), _p(x), _p(y), rows, cols)
    return y


def ref_make_test_case(seed: int, rows: int, cols: int, want_x: bool):
    w = np.zeros((rows, cols), np.int8)
    mask = np.zeros((rows, cols), np.uint8)
    x = np.zeros(cols, np.int8)
    ref().ref_make_test_case(seed, rows, cols, int(want_x), _p(w), _p(mask), _p(x))
    return w, mask, (x if want_x else None)


# ---- the structured-sparse int8 GEMM (the cuSPARSELt backend) -------------------------

def prune24_i8(A: np.ndarray) -> np.ndarray:
    """The build's 2:4 pruning of a dense int8 [m][k] matrix along k (see
    spbo_prune24_i8; the reference's cuSPARSELt STRIP rule is unspecified)."""
    A = np.ascontiguousarray(A, dtype=np.int8)
    m, k = A.shape
    out = np.zeros_like(A)
    lib().spbo_prune24_i8(_p(A), m, k, _p(out))
    return out


def int8_gemm(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    """cpu_int8_gemm (tests/test_cusparselt.cu:16-28): A int8 [m][k], B int8
    [n][k] (column-major [k x n]); returns D int32 [n][m] (column-major [m x n])."""
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    m, k = A.shape
    n = B.shape[0]
    D = np.zeros((n, m), np.int32)
    lib().spbo_int8_gemm(_p(A), _p(B), _p(D), m, k, n)
    return D


# ---- random-init model generator (spb_gen.c) ----------------------------------------

def gen_normals(seed: int, n: int, start: int = 0) -> np.ndarray:
    """The generator's latent N(0,1) values normal(seed, start + i), i < n."""
    out = np.empty(n, np.float32)
    lib().spbo_gen_normals(seed & 0xFFFFFFFFFFFFFFFF, start, n, _p(out))
    return out


def gen_sparse_ternary(seed: int, rows: int, cols: int):
    """(meta, values, gamma) of spb_generate_sparse_ternary: the latent of
    gen_normals packed by python/convert_model.py's recipe (mask_top2,
    kept_sign, pack above) and gamma in the device's summation order."""
    w = gen_normals(seed, rows * cols).reshape(rows, cols)
    mask = mask_top2(w)
    meta, values = pack(kept_sign(w, mask), mask)
    gamma = float(np.float32(lib().spbo_gen_gamma(_p(w), rows, cols)))
    return meta, values, gamma


def gen_normal_bf16(seed: int, n: int, std: float) -> np.ndarray:
    """bf16 bits of spb_generate_normal_bf16 (the embedding)."""
    out = np.empty(n, np.uint16)
    lib().spbo_gen_normal_bf16(seed & 0xFFFFFFFFFFFFFFFF, n, float(std), _p(out))
    return out


def host_random_model(config, seed: int = 0, embed_std: float = 0.02,
                      sub_norms: bool = True) -> dict:
    """The host copy (the layout of spbitnet_amd.model.Model.to_host()) of
    Model.random(config, seed, embed_std=embed_std, sub_norms=sub_norms),
    generated on the CPU: the same per-tensor seeds, latents, packing, gamma
    bits and bf16 embedding, so the oracle can decode the models the GPU
    decodes without a GPU."""
    from spbitnet_amd.weights import seed_for
    c = config
    H, I, kvd = c.hidden_size, c.intermediate_size, c.num_key_value_heads * c.head_dim
    shapes = {"q_proj": (H, H), "k_proj": (kvd, H), "v_proj": (kvd, H), "o_proj": (H, H),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
    out = {"config": c, "layers": []}
    for li in range(c.num_hidden_layers):
        d = {}
        for name in EngineOracle.PROJ:
            rows, cols = shapes[name]
            meta, values, gamma = gen_sparse_ternary(seed_for("model", seed, li, name), rows, cols)
            d[name] = (meta, values, gamma, rows, cols, meta.shape[1], values.shape[1])
        ones = np.ones(H, np.float32)
        d["norms"] = [ones, ones.copy(), ones.copy() if sub_norms else None,
                      np.ones(I, np.float32) if sub_norms else None]
        out["layers"].append(d)
    out["embed"] = gen_normal_bf16(seed_for("model", seed, "embed"), c.vocab_size * H,
                                   embed_std).reshape(c.vocab_size, H)
    out["lm_head"] = None
    out["final_norm"] = np.ones(H, np.float32)
    return out


# ---- decode-step restatement (spb_engine_oracle.c) ---------------------------------

_engine_lib = None


def _elib():
    global _engine_lib
    if _engine_lib is None:
        L = lib()
        L.spbo_engine_new.argtypes = [_P] * 11
        L.spbo_engine_new.restype = _P
        L.spbo_engine_free.argtypes = [_P]
        L.spbo_engine_reset.argtypes = [_P]
        L.spbo_engine_step.argtypes = [_P, _I, _P]
        L.spbo_engine_step.restype = _I
        L.spbo_engine_prefill.argtypes = [_P, _I]
        L.spbo_engine_prefill.restype = _I
        L.spbo_engine_hidden.argtypes = [_P, _P]
        L.spbo_engine_debug.argtypes = [_P, _I, _P]
        L.spbo_engine_debug.restype = _I
        L.spbo_exp_neg.argtypes = [_F]
        L.spbo_exp_neg.restype = _F
        _engine_lib = L
    return _engine_lib


def exp_neg(x: float) -> float:
    return float(np.float32(_elib().spbo_exp_neg(float(x))))


class EngineOracle:
    """CPU decode step of the reference engine (src/inference.cu:126-283) on
    host copies of a model (spbitnet_amd.model.Model.to_host())."""

    PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

    def __init__(self, host: dict, max_seq: int):
        c = host["config"]
        self._keep = []
        nl = len(host["layers"])

        def arr(a, dt):
            a = np.ascontiguousarray(a, dtype=dt)
            self._keep.append(a)
            return a

        metas = (ctypes.c_void_p * (7 * nl))()
        values = (ctypes.c_void_p * (7 * nl))()
        gam = np.zeros(7 * nl, np.float32)
        ms = np.zeros(7 * nl, np.int32)
        vs = np.zeros(7 * nl, np.int32)
        norms = (ctypes.c_void_p * (4 * nl))()
        for l, d in enumerate(host["layers"]):
            for k, p in enumerate(self.PROJ):
                m, v, g, rows, cols, mstr, vstr = d[p]
                metas[7 * l + k] = arr(m, np.uint32).ctypes.data
                values[7 * l + k] = arr(v, np.uint32).ctypes.data
                gam[7 * l + k] = g
                ms[7 * l + k] = mstr
                vs[7 * l + k] = vstr
            for k, t in enumerate(d["norms"]):
                norms[4 * l + k] = None if t is None else arr(t, np.float32).ctypes.data
        self._keep += [metas, values, gam, ms, vs, norms]
        icfg = arr([c.hidden_size, c.num_hidden_layers, c.num_attention_heads,
                    c.num_key_value_heads, c.intermediate_size, c.vocab_size, c.head_dim,
                    max_seq], np.int32)
        fcfg = arr([c.rms_norm_eps, c.rope_theta], np.float32)
        embed = arr(host["embed"], np.uint16)
        lm = None if host["lm_head"] is None else arr(host["lm_head"], np.uint16).ctypes.data
        fn = arr(host["final_norm"], np.float32)
        self.vocab = c.vocab_size
        self.hidden_size = c.hidden_size
        self._e = _elib().spbo_engine_new(icfg.ctypes.data, fcfg.ctypes.data, metas, values,
                                          gam.ctypes.data, ms.ctypes.data, vs.ctypes.data,
                                          norms, embed.ctypes.data, lm, fn.ctypes.data)

    def __del__(self):
        if getattr(self, "_e", None):
            try:
                _elib().spbo_engine_free(self._e)
            except Exception:  # interpreter shutdown: the module is gone
                pass
            self._e = None

    def reset(self):
        _elib().spbo_engine_reset(self._e)

    def step(self, token: int):
        """(argmax, float32 logits) after feeding `token` at the next position."""
        logits = np.empty(self.vocab, np.float32)
        t = _elib().spbo_engine_step(self._e, int(token), _p(logits))
        if t < 0:
            raise ValueError("oracle step: KV cache full or token id out of range")
        return int(t), logits

    def prefill(self, token: int) -> None:
        """A prompt token before the last: the step without the LM head."""
        if _elib().spbo_engine_prefill(self._e, int(token)) < 0:
            raise ValueError("oracle prefill: KV cache full or token id out of range")

    def hidden(self) -> np.ndarray:
        out = np.empty(self.hidden_size, np.float32)
        _elib().spbo_engine_hidden(self._e, _p(out))
        return out

    DEBUG = {"qkv": 0, "attn": 1, "o": 2, "x_mid": 3, "gate_up": 4, "h": 5, "m": 6, "xn": 7}

    def debug(self, name: str) -> np.ndarray:
        """An internal vector of the last step's last layer (see
        spbo_engine_debug)."""
        out = np.empty(4 * (self.hidden_size + 32768), np.float32)
        n = _elib().spbo_engine_debug(self._e, self.DEBUG[name], _p(out))
        return out[:n].copy()

    def generate(self, prompt, n_new: int, eos: int = -1):
        """Greedy generation with the convention of src/main.cpp:133-155."""
        self.reset()
        for t in prompt[:-1]:
            self.prefill(t)
        tok = prompt[-1]
        out = []
        for _ in range(n_new):
            tok, _ = self.step(tok)
            out.append(tok)
            if tok == eos:
                break
        return out

