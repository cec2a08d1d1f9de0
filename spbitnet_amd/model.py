"""Model and decode-engine API over the C ABI, mirroring the reference's
include/spbitnet/model.h (ModelConfig, SparseLinear, TransformerLayer, Model)
and include/spbitnet/inference.h (InferenceEngine): same names and meaning,
torch device tensors in place of raw device pointers.

Weights live in torch tensors (device memory owned by torch); the engine
borrows them, as the reference engine borrows ``const Model&``
(include/spbitnet/inference.h:44), so the Model must outlive its engines.
Activations, the KV cache and the embedding / LM head are bf16.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from .weights import seed_for


@dataclass
class ModelConfig:
    """ModelConfig (reference include/spbitnet/model.h:23-40)."""
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    intermediate_size: int
    vocab_size: int
    max_position_embeddings: int
    head_dim: int = 0
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    bos_token_id: int = 1
    eos_token_id: int = 2
    model_type: str = "bitnet"
    hidden_act: str = "relu2"
    tie_word_embeddings: bool = True

    def __post_init__(self):
        if not self.head_dim:
            self.head_dim = self.hidden_size // self.num_attention_heads

    @staticmethod
    def bitnet_b158_2b4t(max_position_embeddings: int = 4096) -> "ModelConfig":
        """The BitNet b1.58 2B-4T shape (30 layers, hidden 2560, 20 / 5 heads,
        head_dim 128, FFN 6912, vocab 128256, RoPE theta 500000)."""
        return ModelConfig(hidden_size=2560, num_hidden_layers=30, num_attention_heads=20,
                           num_key_value_heads=5, intermediate_size=6912, vocab_size=128256,
                           max_position_embeddings=max_position_embeddings, head_dim=128,
                           rms_norm_eps=1e-5, rope_theta=500000.0, bos_token_id=128000,
                           eos_token_id=128001)

    def c_struct(self) -> _lib.ModelConfigC:
        return _lib.ModelConfigC(self.hidden_size, self.num_hidden_layers,
                                 self.num_attention_heads, self.num_key_value_heads,
                                 self.intermediate_size, self.vocab_size,
                                 self.max_position_embeddings, self.head_dim,
                                 float(self.rms_norm_eps), float(self.rope_theta),
                                 self.bos_token_id, self.eos_token_id)


@dataclass
class SparseLinear:
    """SparseLinear (reference include/spbitnet/model.h:46-60)."""
    meta: torch.Tensor    # int32 [rows, meta_stride]
    values: torch.Tensor  # int32 [rows, values_stride]
    gamma: float
    rows: int
    cols: int
    meta_stride: int
    values_stride: int

    def gpu_bytes(self) -> int:
        return 4 * self.rows * (self.meta_stride + self.values_stride)

    def c_struct(self) -> _lib.SparseLinearC:
        return _lib.SparseLinearC(self.meta.data_ptr(), self.values.data_ptr(),
                                  float(self.gamma), self.rows, self.cols, self.meta_stride,
                                  self.values_stride)


PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass
class TransformerLayer:
    """TransformerLayer (reference include/spbitnet/model.h:63-82)."""
    q_proj: SparseLinear
    k_proj: SparseLinear
    v_proj: SparseLinear
    o_proj: SparseLinear
    gate_proj: SparseLinear
    up_proj: SparseLinear
    down_proj: SparseLinear
    input_layernorm: torch.Tensor           # float32 [hidden]
    post_attention_layernorm: torch.Tensor  # float32 [hidden]
    attn_sub_norm: Optional[torch.Tensor] = None  # float32 [hidden]
    ffn_sub_norm: Optional[torch.Tensor] = None   # float32 [intermediate]

    def c_struct(self) -> _lib.TransformerLayerC:
        def ptr(t):
            return t.data_ptr() if t is not None else None
        return _lib.TransformerLayerC(*[getattr(self, n).c_struct() for n in PROJECTIONS],
                                      ptr(self.input_layernorm),
                                      ptr(self.post_attention_layernorm),
                                      ptr(self.attn_sub_norm), ptr(self.ffn_sub_norm))


@dataclass
class Model:
    """Model (reference include/spbitnet/model.h:88-145): all weights on the
    GPU.  embed_tokens and lm_head are bf16 [vocab, hidden]; lm_head None
    means tied to the embedding (model.h:131-133)."""
    config: ModelConfig
    layers: List[TransformerLayer]
    embed_tokens: torch.Tensor
    final_norm: torch.Tensor
    lm_head_weight: Optional[torch.Tensor] = None
    _keep: list = field(default_factory=list, repr=False)

    def lm_head(self) -> torch.Tensor:
        return self.lm_head_weight if self.lm_head_weight is not None else self.embed_tokens

    def layer(self, i: int) -> TransformerLayer:
        return self.layers[i]

    def total_gpu_bytes(self) -> int:
        n = sum(getattr(l, p).gpu_bytes() for l in self.layers for p in PROJECTIONS)
        n += self.embed_tokens.numel() * 2 + self.final_norm.numel() * 4
        if self.lm_head_weight is not None:
            n += self.lm_head_weight.numel() * 2
        for l in self.layers:
            for t in (l.input_layernorm, l.post_attention_layernorm, l.attn_sub_norm,
                      l.ffn_sub_norm):
                if t is not None:
                    n += t.numel() * 4
        return n

    @staticmethod
    def random(config: ModelConfig, seed: int = 0, device="cuda", embed_std: float = 0.02,
               sub_norms: bool = True) -> "Model":
        """Random-init model generated on the device: every projection from
        latent W ~ N(0,1) through the 2:4 top-2 mask and ternary signs
        (convert_model.py's recipe), embedding ~ N(0, embed_std^2) in bf16
        (tied LM head), every RMSNorm weight 1.0."""
        c = config
        dev = torch.device(device)
        H, I, kvd = c.hidden_size, c.intermediate_size, c.num_key_value_heads * c.head_dim
        shapes = {"q_proj": (H, H), "k_proj": (kvd, H), "v_proj": (kvd, H), "o_proj": (H, H),
                  "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
        L = _lib.load()
        stream = torch.cuda.current_stream(dev).cuda_stream or None
        gammas = torch.zeros(c.num_hidden_layers * len(PROJECTIONS), dtype=torch.float32,
                             device=dev)
        raw = []
        for li in range(c.num_hidden_layers):
            row = {}
            for pi, name in enumerate(PROJECTIONS):
                rows, cols = shapes[name]
                ms, vs = cols // 32, cols // 64
                meta = torch.empty((rows, ms), dtype=torch.int32, device=dev)
                values = torch.empty((rows, vs), dtype=torch.int32, device=dev)
                g = gammas[li * len(PROJECTIONS) + pi:]
                _lib.check(L.spb_generate_sparse_ternary(
                    seed_for("model", seed, li, name) & 0xFFFFFFFFFFFFFFFF, rows, cols,
                    meta.data_ptr(), values.data_ptr(), ms, vs, g.data_ptr(), None, stream),
                    "spb_generate_sparse_ternary")
                row[name] = (meta, values, rows, cols, ms, vs)
            raw.append(row)
        embed = torch.empty((c.vocab_size, H), dtype=torch.bfloat16, device=dev)
        _lib.check(L.spb_generate_normal_bf16(seed_for("model", seed, "embed") & 0xFFFFFFFFFFFFFFFF,
                                              embed.numel(), float(embed_std), embed.data_ptr(),
                                              stream), "spb_generate_normal_bf16")
        g_host = gammas.cpu().numpy()
        layers = []
        for li, row in enumerate(raw):
            lin = {}
            for pi, name in enumerate(PROJECTIONS):
                meta, values, rows, cols, ms, vs = row[name]
                lin[name] = SparseLinear(meta, values, float(g_host[li * len(PROJECTIONS) + pi]),
                                         rows, cols, ms, vs)
            ones_h = torch.ones(H, dtype=torch.float32, device=dev)
            layers.append(TransformerLayer(
                **lin, input_layernorm=ones_h, post_attention_layernorm=ones_h.clone(),
                attn_sub_norm=ones_h.clone() if sub_norms else None,
                ffn_sub_norm=torch.ones(I, dtype=torch.float32, device=dev) if sub_norms else None))
        return Model(config, layers, embed, torch.ones(H, dtype=torch.float32, device=dev))

    def engine_args(self):
        """(config, layer array, embed, lm_head, final_norm) for spb_engine_create."""
        layers = (_lib.TransformerLayerC * self.config.num_hidden_layers)(
            *[l.c_struct() for l in self.layers])
        lm = self.lm_head_weight.data_ptr() if self.lm_head_weight is not None else None
        return (self.config.c_struct(), layers, self.embed_tokens.data_ptr(), lm,
                self.final_norm.data_ptr())

    @staticmethod
    def load(model_dir: str, device="cuda") -> "Model":
        """Model::load (include/spbitnet/model.h:103)."""
        return load_model(model_dir, device)

    def save(self, model_dir: str) -> None:
        save_model(self, model_dir)

    def to_host(self) -> dict:
        """Host (numpy) copies of every weight, for the CPU oracle."""
        def npf(t):
            return None if t is None else t.detach().cpu().numpy()
        out = {"config": self.config, "layers": []}
        for l in self.layers:
            d = {}
            for p in PROJECTIONS:
                s = getattr(l, p)
                d[p] = (s.meta.cpu().numpy().view(np.uint32), s.values.cpu().numpy().view(np.uint32),
                        s.gamma, s.rows, s.cols, s.meta_stride, s.values_stride)
            d["norms"] = [npf(l.input_layernorm), npf(l.post_attention_layernorm),
                          npf(l.attn_sub_norm), npf(l.ffn_sub_norm)]
            out["layers"].append(d)
        out["embed"] = self.embed_tokens.cpu().view(torch.int16).numpy().view(np.uint16)
        out["lm_head"] = (None if self.lm_head_weight is None else
                          self.lm_head_weight.cpu().view(torch.int16).numpy().view(np.uint16))
        out["final_norm"] = npf(self.final_norm)
        return out


# ---- on-disk format (python/convert_model.py; docs/compression_format.md sec. 4) ----

_NORM_NAMES = (("input_layernorm", "input_layernorm"),
               ("post_attention_layernorm", "post_attention_layernorm"),
               ("attn_sub_norm", "self_attn.attn_sub_norm"),
               ("ffn_sub_norm", "mlp.ffn_sub_norm"))
_PROJ_NAMES = {"q_proj": "self_attn.q_proj", "k_proj": "self_attn.k_proj",
               "v_proj": "self_attn.v_proj", "o_proj": "self_attn.o_proj",
               "gate_proj": "mlp.gate_proj", "up_proj": "mlp.up_proj",
               "down_proj": "mlp.down_proj"}
_CONFIG_KEYS = ("model_type", "hidden_size", "num_hidden_layers", "num_attention_heads",
                "num_key_value_heads", "intermediate_size", "vocab_size",
                "max_position_embeddings", "rms_norm_eps", "rope_theta", "head_dim",
                "hidden_act", "tie_word_embeddings", "bos_token_id", "eos_token_id")


def save_model(model: "Model", model_dir: str) -> None:
    """Write a model in the reference's converted-model layout: config.json,
    manifest.json and weights/*.meta|.values|.bin (export_sparse_layer and
    the export loop of python/convert_model.py).  The embedding and a separate
    LM head are written as float16, the reference's storage type."""
    import json
    import os
    c = model.config
    os.makedirs(os.path.join(model_dir, "weights"), exist_ok=True)
    cfg = {k: getattr(c, k) for k in _CONFIG_KEYS}
    cfg["tie_word_embeddings"] = model.lm_head_weight is None
    with open(os.path.join(model_dir, "config.json"), "w") as f:
        json.dump(cfg, f, indent=2)
    weights = {}

    def write(name, arr):
        rel = f"weights/{name}"
        np.ascontiguousarray(arr).tofile(os.path.join(model_dir, rel))
        return rel

    def dense16(name, t):
        a = t.detach().to(torch.float16).cpu().numpy()
        weights[name] = {"file": write(name + ".bin", a), "dtype": "float16",
                         "shape": list(a.shape), "nbytes": int(a.nbytes)}

    def f32(name, t):
        a = t.detach().float().cpu().numpy()
        weights[name] = {"file": write(name + ".bin", a), "dtype": "float32",
                         "shape": list(a.shape), "nbytes": int(a.nbytes)}

    dense16("embed_tokens", model.embed_tokens)
    f32("norm", model.final_norm)
    if model.lm_head_weight is None:
        weights["lm_head"] = {"tied_to": "embed_tokens", "dtype": "tied"}
    else:
        dense16("lm_head", model.lm_head_weight)
    for li, L in enumerate(model.layers):
        for attr, name in _NORM_NAMES:
            t = getattr(L, attr)
            if t is not None:
                f32(f"layers.{li}.{name}", t)
        for attr, name in _PROJ_NAMES.items():
            s = getattr(L, attr)
            full = f"layers.{li}.{name}"
            m = s.meta.cpu().numpy().view(np.uint32)
            v = s.values.cpu().numpy().view(np.uint32)
            weights[full] = {"meta_file": write(full + ".meta", m),
                             "values_file": write(full + ".values", v),
                             "dtype": "sparse_ternary", "shape": [s.rows, s.cols],
                             "meta_stride": s.meta_stride, "values_stride": s.values_stride,
                             "gamma": float(s.gamma), "meta_nbytes": int(m.nbytes),
                             "values_nbytes": int(v.nbytes)}
    with open(os.path.join(model_dir, "manifest.json"), "w") as f:
        json.dump({"format_version": 1, "weights": weights}, f, indent=1)


def load_model(model_dir: str, device="cuda") -> "Model":
    """Model::load (src/model.cu:180-311) in Python: reads the converted-model
    layout into torch device tensors; the fp16 embedding / LM head become
    bf16."""
    import json
    import os
    dev = torch.device(device)
    with open(os.path.join(model_dir, "config.json")) as f:
        cj = json.load(f)
    with open(os.path.join(model_dir, "manifest.json")) as f:
        w = json.load(f)["weights"]
    nh = cj["num_attention_heads"]
    c = ModelConfig(hidden_size=cj["hidden_size"], num_hidden_layers=cj["num_hidden_layers"],
                    num_attention_heads=nh,
                    num_key_value_heads=cj.get("num_key_value_heads", nh),
                    intermediate_size=cj["intermediate_size"], vocab_size=cj["vocab_size"],
                    max_position_embeddings=cj["max_position_embeddings"],
                    head_dim=cj.get("head_dim", cj["hidden_size"] // nh),
                    rms_norm_eps=cj.get("rms_norm_eps", 1e-5),
                    rope_theta=cj.get("rope_theta", 10000.0),
                    bos_token_id=cj.get("bos_token_id", 1), eos_token_id=cj.get("eos_token_id", 2),
                    model_type=cj.get("model_type", "bitnet"),
                    hidden_act=cj.get("hidden_act", "relu2"),
                    tie_word_embeddings=cj.get("tie_word_embeddings", False))

    def raw(rel, dtype, count):
        a = np.fromfile(os.path.join(model_dir, rel), dtype=dtype)
        if a.size != count:
            raise ValueError(f"{rel}: {a.size} elements, expected {count}")
        return a

    def f32(name, n):
        if name not in w:
            return None
        return torch.from_numpy(raw(w[name]["file"], "<f4", n).copy()).to(dev)

    def dense16(e, n):
        if e.get("dtype") == "bfloat16":
            bits = raw(e["file"], "<u2", n).view(np.int16)
            return torch.from_numpy(bits.copy()).view(torch.bfloat16).reshape(c.vocab_size, c.hidden_size).to(dev)
        a = raw(e["file"], "<f2", n)
        return torch.from_numpy(a.copy()).to(dev).to(torch.bfloat16).reshape(c.vocab_size, c.hidden_size)

    H, I = c.hidden_size, c.intermediate_size
    kvd = c.num_key_value_heads * c.head_dim
    shapes = {"q_proj": (H, H), "k_proj": (kvd, H), "v_proj": (kvd, H), "o_proj": (H, H),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
    embed = dense16(w["embed_tokens"], c.vocab_size * H)
    lm = None
    if "lm_head" in w and w["lm_head"].get("dtype") != "tied":
        lm = dense16(w["lm_head"], c.vocab_size * H)
    layers = []
    for li in range(c.num_hidden_layers):
        lin = {}
        for attr, name in _PROJ_NAMES.items():
            e = w[f"layers.{li}.{name}"]
            rows, cols = e["shape"]
            if (rows, cols) != shapes[attr]:
                raise ValueError(f"layers.{li}.{name}: shape {rows}x{cols}, expected {shapes[attr]}")
            for key in ("meta_stride", "values_stride", "gamma"):
                if key not in e:  # required, as in src/model.cu:107-109
                    raise ValueError(f"layers.{li}.{name}: manifest entry lacks {key}")
            ms, vs = int(e["meta_stride"]), int(e["values_stride"])
            if ms < (cols + 31) // 32 or vs < (cols + 63) // 64:
                raise ValueError(f"layers.{li}.{name}: strides {ms}/{vs} do not cover a row of "
                                 f"{cols} columns")
            m = torch.from_numpy(raw(e["meta_file"], "<u4", rows * ms).view(np.int32).reshape(rows, ms).copy())
            v = torch.from_numpy(raw(e["values_file"], "<u4", rows * vs).view(np.int32).reshape(rows, vs).copy())
            lin[attr] = SparseLinear(m.to(dev), v.to(dev), float(np.float32(e["gamma"])), rows, cols,
                                     ms, vs)
        norms = {attr: f32(f"layers.{li}.{name}", I if attr == "ffn_sub_norm" else H)
                 for attr, name in _NORM_NAMES}
        layers.append(TransformerLayer(**lin, **norms))
    return Model(c, layers, embed, f32("norm", H), lm)


class NativeModel:
    """A model loaded by the library's own loader (spb_model_load, C++):
    the form a C++ host uses; device memory owned by the library."""

    def __init__(self, model_dir: str):
        self._L = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(self._L.spb_model_load(model_dir.encode(), ctypes.byref(h)), "spb_model_load")
        self._h = h
        cfg = _lib.ModelConfigC()
        layers = ctypes.c_void_p()
        emb, lm, fn, nbytes = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_size_t()
        _lib.check(self._L.spb_model_info(self._h, ctypes.byref(cfg), ctypes.byref(layers),
                                          ctypes.byref(emb), ctypes.byref(lm), ctypes.byref(fn),
                                          ctypes.byref(nbytes)), "spb_model_info")
        self._cfg, self._layers_ptr = cfg, layers.value
        self._embed, self._lm, self._final = emb.value, lm.value, fn.value
        self.gpu_bytes = nbytes.value
        self.config = ModelConfig(hidden_size=cfg.hidden_size,
                                  num_hidden_layers=cfg.num_hidden_layers,
                                  num_attention_heads=cfg.num_attention_heads,
                                  num_key_value_heads=cfg.num_key_value_heads,
                                  intermediate_size=cfg.intermediate_size,
                                  vocab_size=cfg.vocab_size,
                                  max_position_embeddings=cfg.max_position_embeddings,
                                  head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps,
                                  rope_theta=cfg.rope_theta, bos_token_id=cfg.bos_token_id,
                                  eos_token_id=cfg.eos_token_id)

    def engine_args(self):
        return (self._cfg, ctypes.c_void_p(self._layers_ptr), self._embed, self._lm, self._final)

    def close(self):
        if getattr(self, "_h", None):
            self._L.spb_model_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


class InferenceEngine:
    """InferenceEngine (reference include/spbitnet/inference.h:23-70) over the
    HIP decode engine: forward() one token at a time, reset(), seq_len(), plus
    generate(), which runs a whole greedy generation on the device."""

    def __init__(self, model: Model, max_seq: Optional[int] = None, stream=None):
        self.model = model
        c = model.config
        self.max_seq = int(max_seq or c.max_position_embeddings)
        self._L = _lib.load()
        cfg, layers, embed, lm, final = model.engine_args()
        self._cfg, self._layers = cfg, layers
        h = ctypes.c_void_p()
        _lib.check(self._L.spb_engine_create(ctypes.byref(cfg), layers, embed, lm, final,
                                             self.max_seq, ctypes.byref(h)), "spb_engine_create")
        self._h = h
        self._stream = stream if stream is not None else torch.cuda.current_stream()
        _lib.check(self._L.spb_engine_set_stream(self._h, self._stream.cuda_stream or None),
                   "spb_engine_set_stream")
        lp, tp = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(self._L.spb_engine_buffers(self._h, ctypes.byref(lp), ctypes.byref(tp)),
                   "spb_engine_buffers")
        self._logits_ptr = lp.value
        self._logits = torch.empty(c.vocab_size, dtype=torch.float32,
                                   device=torch.device("cuda", torch.cuda.current_device()))

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.spb_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def reset(self) -> None:
        _lib.check(self._L.spb_engine_reset(self._h), "spb_engine_reset")

    def seq_len(self) -> int:
        return self._L.spb_engine_seq_len(self._h)

    def forward(self, token_id: int) -> torch.Tensor:
        """Logits (float32 [vocab], on the device) for the next token."""
        _lib.check(self._L.spb_engine_forward(self._h, int(token_id), None),
                   "spb_engine_forward")
        _lib.memcpy_d2d(self._logits.data_ptr(), self._logits_ptr, self._logits.numel() * 4,
                        self._stream.cuda_stream or None)
        return self._logits

    def generate(self, prompt: Sequence[int], n_new: int, stop_at_eos: bool = True) -> List[int]:
        """Greedy generation (src/main.cpp:133-155): prefill prompt[:-1], then
        n_new steps from the last prompt token."""
        p = (ctypes.c_int * len(prompt))(*[int(t) for t in prompt])
        out = (ctypes.c_int * max(1, n_new))()
        got = ctypes.c_int(0)
        _lib.check(self._L.spb_engine_generate(self._h, p, len(prompt), int(n_new),
                                               1 if stop_at_eos else 0, out, ctypes.byref(got)),
                   "spb_engine_generate")
        return list(out[:got.value])

    def set_prefill_batch(self, min_tokens: int) -> None:
        """generate() prefills a prompt with at least min_tokens tokens before
        its last in batches through the layers (matrix-core GEMM; the same KV
        cache and tokens as one step per token); 0 = one step per token."""
        _lib.check(self._L.spb_engine_set_prefill_batch(self._h, int(min_tokens)),
                   "spb_engine_set_prefill_batch")

    def decode_steps(self, steps: int) -> None:
        """Enqueue `steps` more greedy steps (no host synchronisation)."""
        _lib.check(self._L.spb_engine_decode_steps(self._h, int(steps)),
                   "spb_engine_decode_steps")


class BatchInferenceEngine:
    """Greedy decode of several independent sequences per step on the HIP
    batched engine (spb_batch_engine_*).  No reference counterpart: the
    reference's InferenceEngine decodes one sequence; each sequence's tokens
    here equal InferenceEngine.generate on that sequence alone."""

    def __init__(self, model, max_seq: int, batch: int, stream=None):
        self.model = model
        self.max_seq = int(max_seq)
        self.batch = int(batch)
        self._L = _lib.load()
        cfg, layers, embed, lm, final = model.engine_args()
        self._cfg, self._layers = cfg, layers
        h = ctypes.c_void_p()
        _lib.check(self._L.spb_batch_engine_create(ctypes.byref(cfg), layers, embed, lm, final,
                                                   self.max_seq, self.batch, ctypes.byref(h)),
                   "spb_batch_engine_create")
        self._h = h
        self._stream = stream if stream is not None else torch.cuda.current_stream()
        _lib.check(self._L.spb_batch_engine_set_stream(self._h, self._stream.cuda_stream or None),
                   "spb_batch_engine_set_stream")

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.spb_batch_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def generate(self, prompts: Sequence[Sequence[int]], n_new: int,
                 stop_at_eos: bool = True) -> List[List[int]]:
        """Greedy generation of len(prompts) <= batch sequences at once; one
        token list per sequence (src/main.cpp:133-155 per sequence)."""
        flat = [int(t) for p in prompts for t in p]
        lens = (ctypes.c_int * len(prompts))(*[len(p) for p in prompts])
        fp = (ctypes.c_int * max(1, len(flat)))(*flat)
        out = (ctypes.c_int * max(1, len(prompts) * n_new))()
        got = (ctypes.c_int * len(prompts))()
        _lib.check(self._L.spb_batch_engine_generate(self._h, fp, lens, len(prompts), int(n_new),
                                                     1 if stop_at_eos else 0, out, got),
                   "spb_batch_engine_generate")
        return [list(out[b * n_new: b * n_new + got[b]]) for b in range(len(prompts))]

    def decode_steps(self, steps: int) -> None:
        """Enqueue `steps` more batched steps (no host synchronisation)."""
        _lib.check(self._L.spb_batch_engine_decode_steps(self._h, int(steps)),
                   "spb_batch_engine_decode_steps")

    def token_buffer(self) -> torch.Tensor:
        """A copy of the device token buffer, int32 [batch][max_seq + 1]:
        sequence b's prompt, then one token per decode step at its
        positions (what decode_steps appends)."""
        tp = ctypes.c_void_p()
        _lib.check(self._L.spb_batch_engine_buffers(self._h, None, ctypes.byref(tp)),
                   "spb_batch_engine_buffers")
        out = torch.empty((self.batch, self.max_seq + 1), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        _lib.memcpy_d2d(out.data_ptr(), tp.value, out.numel() * 4, None)
        torch.cuda.synchronize()
        return out

    def last_logits(self) -> torch.Tensor:
        """A copy of the last step's float32 logits, [batch][vocab].  Each
        sequence's argmax row holds the bs=1 engine's value bit for bit; the
        other rows are the matrix-core products, within the LM head's error
        bound of it (spb_batch_engine_create in csrc/engine.hip)."""
        lp = ctypes.c_void_p()
        _lib.check(self._L.spb_batch_engine_buffers(self._h, ctypes.byref(lp), None),
                   "spb_batch_engine_buffers")
        V = self.model.config.vocab_size
        out = torch.empty((self.batch, V), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        _lib.memcpy_d2d(out.data_ptr(), lp.value, out.numel() * 4, None)
        torch.cuda.synchronize()
        return out
