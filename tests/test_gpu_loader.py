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
