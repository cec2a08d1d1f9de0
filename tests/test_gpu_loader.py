"""The library's native loader (spb_model_load, the reference's Model::load,
src/model.cu:180-311) and the Python loader on a written model: identical
weights, identical greedy tokens, bit-exact against the oracle."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _cfg():
    from spbitnet_amd.model import ModelConfig
    return ModelConfig(hidden_size=512, num_hidden_layers=2, num_attention_heads=8,
                       num_key_value_heads=2, intermediate_size=1536, vocab_size=3000,
                       max_position_embeddings=512, head_dim=64, rope_theta=500000.0,
                       bos_token_id=1, eos_token_id=2)


def test_native_and_python_loaders_agree(gpu, tmp_path):
    from spbitnet_amd.model import InferenceEngine, Model, NativeModel, load_model
    cfg = _cfg()
    src = Model.random(cfg, seed=77)
    src.save(str(tmp_path))
    py = load_model(str(tmp_path))
    nat = NativeModel(str(tmp_path))
    assert nat.config.hidden_size == 512 and nat.config.num_key_value_heads == 2
    assert nat.gpu_bytes > 0
    prompt = [int(t) for t in np.random.default_rng(1).integers(0, cfg.vocab_size, 12)]
    e1 = InferenceEngine(py, max_seq=128)
    e2 = InferenceEngine(nat, max_seq=128)
    t1 = e1.generate(prompt, 48, stop_at_eos=False)
    t2 = e2.generate(prompt, 48, stop_at_eos=False)
    assert t1 == t2
    assert t1 == O.EngineOracle(py.to_host(), 128).generate(prompt, 48)
    e1.close()
    e2.close()
    nat.close()


def test_native_loader_errors(gpu, tmp_path):
    from spbitnet_amd import _lib
    from spbitnet_amd.model import Model, NativeModel
    cfg = _cfg()
    Model.random(cfg, seed=1).save(str(tmp_path))
    meta = tmp_path / "weights" / "layers.1.mlp.down_proj.meta"
    data = meta.read_bytes()
    meta.write_bytes(data[:-4])
    with pytest.raises(_lib.SpbError, match="down_proj"):
        NativeModel(str(tmp_path))
    meta.write_bytes(data)
    m = json.load(open(tmp_path / "manifest.json"))
    del m["weights"]["layers.0.self_attn.k_proj"]
    json.dump(m, open(tmp_path / "manifest.json", "w"))
    with pytest.raises(_lib.SpbError, match="k_proj"):
        NativeModel(str(tmp_path))
    (tmp_path / "manifest.json").write_text("{ not json")
    with pytest.raises(_lib.SpbError, match="manifest.json"):
        NativeModel(str(tmp_path))
    with pytest.raises(_lib.SpbError, match="config.json"):
        NativeModel(str(tmp_path / "missing"))


FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "loader_model")


def test_native_loader_reference_fixture(gpu):
    """The native loader (spb_model_load) on the directory of the reference's
    loader test (tests/test_model_loader.cu:52-191), with that test's
    expectations (:199-284) and the device words its pattern fixes; an engine
    on it is refused (hidden 8 is not a multiple of 128) before any launch."""
    import ctypes
    from spbitnet_amd import _lib
    from spbitnet_amd.model import InferenceEngine, NativeModel
    nat = NativeModel(FIXTURE)
    c = nat.config
    assert (c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads,
            c.intermediate_size, c.vocab_size, c.head_dim) == (8, 1, 1, 1, 16, 32, 8)
    assert nat._lm is None and nat._embed and nat._final  # tied LM head
    assert nat.gpu_bytes > 0
    layer = ctypes.cast(nat._layers_ptr, ctypes.POINTER(_lib.TransformerLayerC))[0]
    assert layer.input_layernorm and layer.post_attention_layernorm
    assert not layer.attn_sub_norm and not layer.ffn_sub_norm
    q, g, d = layer.q_proj, layer.gate_proj, layer.down_proj
    assert (q.rows, q.cols, q.gamma) == (8, 8, 0.5)
    assert (g.rows, g.cols) == (16, 8) and (d.rows, d.cols) == (8, 16)

    def words(ptr, n):
        t = torch.empty(n, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        _lib.memcpy_d2d(t.data_ptr(), ptr, 4 * n, None)
        torch.cuda.synchronize()
        return t.cpu().numpy().view(np.uint32)

    assert (words(q.meta, 8) == 0x33).all() and (words(q.values, 8) == 0xA).all()
    assert (words(d.meta, 8) == 0x3333).all() and (words(d.values, 8) == 0xAA).all()
    emb = torch.empty(32 * 8, dtype=torch.int16, device="cuda")
    _lib.memcpy_d2d(emb.data_ptr(), nat._embed, 32 * 8 * 2, None)
    torch.cuda.synchronize()
    assert (emb.view(torch.bfloat16).float().cpu() == 1.0).all()  # fp16 1.0 -> bf16 1.0
    with pytest.raises(_lib.SpbError):
        InferenceEngine(nat, max_seq=16)
    nat.close()


def test_native_loader_requires_strides_and_gamma(gpu, tmp_path):
    """meta_stride, values_stride and gamma are required (src/model.cu:107-109)
    and the strides must cover a row: the native loader refuses the manifest
    on the host, naming the tensor."""
    import shutil
    from spbitnet_amd import _lib
    from spbitnet_amd.model import NativeModel
    cases = [("layers.0.mlp.down_proj", "meta_stride", None),
             ("layers.0.mlp.down_proj", "values_stride", None),
             ("layers.0.self_attn.o_proj", "gamma", None),
             ("layers.0.mlp.down_proj", "meta_stride", 0),
             ("layers.0.self_attn.q_proj", "values_stride", 0)]
    for i, (name, key, val) in enumerate(cases):
        d = tmp_path / str(i)
        shutil.copytree(FIXTURE, d)
        man = json.load(open(d / "manifest.json"))
        if val is None:
            del man["weights"][name][key]
        else:
            man["weights"][name][key] = val
        json.dump(man, open(d / "manifest.json", "w"))
        print(f"native loader without {name}.{key}", flush=True)
        with pytest.raises(_lib.SpbError, match=name):
            NativeModel(str(d))
