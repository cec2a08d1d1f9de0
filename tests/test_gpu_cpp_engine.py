"""The reference's C++ model / engine API (include/spbitnet/model.h,
inference.h) in a separate C++ host program (tests/cpp/engine_api.cpp, built
by __graft_entry__.build()): it loads a written model directory through the
library's native loader and its greedy tokens equal the Python engine's and
the oracle's."""
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "engine_api")


def test_cpp_engine_program(gpu, tmp_path):
    from spbitnet_amd.model import InferenceEngine, Model, ModelConfig, load_model
    assert os.path.exists(EXE), "tests/cpp/engine_api is not built (run __graft_entry__.build())"
    cfg = ModelConfig(hidden_size=512, num_hidden_layers=2, num_attention_heads=8,
                      num_key_value_heads=2, intermediate_size=1536, vocab_size=2048,
                      max_position_embeddings=512, head_dim=64, rope_theta=500000.0)
    Model.random(cfg, seed=123).save(str(tmp_path))
    prompt = [int(t) for t in np.random.default_rng(7).integers(0, cfg.vocab_size, 9)]
    print("running the C++ program", flush=True)
    r = subprocess.run([EXE, str(tmp_path), "32"] + [str(t) for t in prompt],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    line = [l for l in r.stdout.splitlines() if l.startswith("tokens")][0]
    cpp_tokens = [int(t) for t in line.split()[1:]]
    assert "seq_len 9" in r.stdout
    model = load_model(str(tmp_path))
    eng = InferenceEngine(model, max_seq=256)
    assert cpp_tokens == eng.generate(prompt, 32, stop_at_eos=False)
    assert cpp_tokens == O.EngineOracle(model.to_host(), 256).generate(prompt, 32)
    eng.close()
