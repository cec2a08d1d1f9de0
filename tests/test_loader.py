"""The converted-model layout (python/convert_model.py; docs/compression_format.md
section 4): writer and Python loader round trip on the CPU, and the layout
the files take (names, dtypes, sizes) as the reference loader
(src/model.cu:180-311) expects it."""
import json
import os

import numpy as np
import torch

from forward64 import host_model
from spbitnet_amd.model import (Model, ModelConfig, SparseLinear, TransformerLayer, load_model,
                                save_model)

PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _cpu_model(cfg, seed=0, sub_norms=True):
    h = host_model(cfg, seed=seed, sub_norms=sub_norms, norm_jitter=0.1)
    layers = []
    for d in h["layers"]:
        lin = {p: SparseLinear(torch.from_numpy(d[p][0].view(np.int32).copy()),
                               torch.from_numpy(d[p][1].view(np.int32).copy()),
                               float(np.float32(d[p][2])), d[p][3], d[p][4], d[p][5], d[p][6])
               for p in PROJ}
        n = [None if t is None else torch.from_numpy(t.copy()) for t in d["norms"]]
        layers.append(TransformerLayer(**lin, input_layernorm=n[0], post_attention_layernorm=n[1],
                                       attn_sub_norm=n[2], ffn_sub_norm=n[3]))
    embed = torch.from_numpy(h["embed"].view(np.int16).copy()).view(torch.bfloat16)
    return Model(cfg, layers, embed, torch.from_numpy(h["final_norm"].copy()))


def _cfg():
    return ModelConfig(hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
                       num_key_value_heads=2, intermediate_size=512, vocab_size=300,
                       max_position_embeddings=512, head_dim=64, rope_theta=500000.0,
                       bos_token_id=1, eos_token_id=2)


def test_layout_matches_reference_loader(tmp_path):
    cfg = _cfg()
    m = _cpu_model(cfg)
    save_model(m, str(tmp_path))
    c = json.load(open(tmp_path / "config.json"))
    for k in ("hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
              "intermediate_size", "vocab_size", "max_position_embeddings", "rms_norm_eps",
              "rope_theta", "head_dim", "bos_token_id", "eos_token_id"):
        assert k in c
    assert c["tie_word_embeddings"] is True
    w = json.load(open(tmp_path / "manifest.json"))["weights"]
    assert w["lm_head"] == {"tied_to": "embed_tokens", "dtype": "tied"}
    e = w["embed_tokens"]
    assert e["dtype"] == "float16" and e["shape"] == [300, 256]
    assert os.path.getsize(tmp_path / e["file"]) == 300 * 256 * 2
    q = w["layers.1.self_attn.q_proj"]
    assert q["dtype"] == "sparse_ternary" and q["shape"] == [256, 256]
    assert q["meta_stride"] == 8 and q["values_stride"] == 4
    assert os.path.getsize(tmp_path / q["meta_file"]) == 256 * 8 * 4 == q["meta_nbytes"]
    assert os.path.getsize(tmp_path / q["values_file"]) == 256 * 4 * 4 == q["values_nbytes"]
    assert w["layers.0.mlp.ffn_sub_norm"]["shape"] == [512]
    assert "layers.0.self_attn.attn_sub_norm" in w and "layers.0.post_attention_layernorm" in w
    assert "norm" in w


def test_round_trip(tmp_path):
    cfg = _cfg()
    m = _cpu_model(cfg, seed=3)
    save_model(m, str(tmp_path))
    r = load_model(str(tmp_path), device="cpu")
    assert r.config.hidden_size == 256 and r.config.num_key_value_heads == 2
    assert r.lm_head_weight is None
    for a, b in zip(m.layers, r.layers):
        for p in PROJ:
            x, y = getattr(a, p), getattr(b, p)
            assert torch.equal(x.meta, y.meta) and torch.equal(x.values, y.values)
            assert x.gamma == y.gamma and (x.rows, x.cols) == (y.rows, y.cols)
        for n in ("input_layernorm", "post_attention_layernorm", "attn_sub_norm", "ffn_sub_norm"):
            assert torch.equal(getattr(a, n), getattr(b, n))
    # bf16 -> fp16 file -> bf16: exact for every value fp16 represents normally
    e16 = m.embed_tokens.float().to(torch.float16).to(torch.bfloat16)
    assert torch.equal(r.embed_tokens, e16)
    assert torch.equal(r.final_norm, m.final_norm)


def test_round_trip_without_sub_norms(tmp_path):
    cfg = _cfg()
    m = _cpu_model(cfg, seed=4, sub_norms=False)
    save_model(m, str(tmp_path))
    r = load_model(str(tmp_path), device="cpu")
    assert r.layers[0].attn_sub_norm is None and r.layers[1].ffn_sub_norm is None


FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "loader_model")


def test_reference_loader_fixture():
    """The directory the reference's loader test writes (create_test_model,
    tests/test_model_loader.cu:52-191) read by the Python loader, with that
    test's expectations (:199-284) and the packed words its pattern fixes:
    {+1, -1, 0, 0} groups are bitmap 0x3 and signs 0b10 per group."""
    m = load_model(FIXTURE, device="cpu")
    c = m.config
    assert (c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads,
            c.intermediate_size, c.vocab_size, c.head_dim) == (8, 1, 1, 1, 16, 32, 8)
    assert c.hidden_act == "relu2" and c.tie_word_embeddings
    assert m.lm_head_weight is None and m.lm_head() is m.embed_tokens  # tied
    assert torch.equal(m.embed_tokens.float(), torch.ones(32, 8))
    assert torch.equal(m.final_norm, torch.ones(8))
    L = m.layers[0]
    assert torch.equal(L.input_layernorm, torch.ones(8))
    assert torch.equal(L.post_attention_layernorm, torch.ones(8))
    assert L.attn_sub_norm is None and L.ffn_sub_norm is None
    assert (L.q_proj.rows, L.q_proj.cols, L.q_proj.gamma) == (8, 8, 0.5)
    assert (L.gate_proj.rows, L.gate_proj.cols) == (16, 8)
    assert (L.down_proj.rows, L.down_proj.cols) == (8, 16)
    assert (L.q_proj.meta.view(-1) == 0x33).all() and (L.q_proj.values.view(-1) == 0xA).all()
    assert (L.down_proj.meta.view(-1) == 0x3333).all()
    assert (L.down_proj.values.view(-1) == 0xAA).all()
    # unpacked rows are +1, -1, 0, 0 repeated
    from spbitnet_amd import weights as Wt
    dense = Wt.unpack(L.down_proj.meta.numpy().view(np.uint32),
                      L.down_proj.values.numpy().view(np.uint32), 8, 16)
    assert (dense == np.tile(np.array([1, -1, 0, 0], np.int8), (8, 4))).all()
    assert m.total_gpu_bytes() > 0


def _fixture_copy(tmp_path, edit):
    import shutil
    d = tmp_path / "model"
    shutil.copytree(FIXTURE, d)
    man = json.load(open(d / "manifest.json"))
    edit(man["weights"])
    json.dump(man, open(d / "manifest.json", "w"))
    return str(d)


def test_loader_rejects_missing_or_short_strides(tmp_path):
    """meta_stride, values_stride and gamma are required (src/model.cu:107-109
    reads them with entry.at()) and the strides must cover a row; a manifest
    that understates them is rejected before any weight reaches a kernel."""
    import pytest
    cases = [
        ("layers.0.mlp.down_proj", "meta_stride", None),
        ("layers.0.mlp.down_proj", "values_stride", None),
        ("layers.0.self_attn.o_proj", "gamma", None),
        ("layers.0.mlp.down_proj", "meta_stride", 0),
        ("layers.0.self_attn.q_proj", "values_stride", 0),
    ]
    for i, (name, key, val) in enumerate(cases):
        def edit(w):
            if val is None:
                del w[name][key]
            else:
                w[name][key] = val
        d = _fixture_copy(tmp_path / str(i), edit)
        with pytest.raises(ValueError, match=name):
            load_model(d, device="cpu")
