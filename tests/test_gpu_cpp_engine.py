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


BITLINEAR_EXE = os.path.join(ROOT, "tests", "cpp", "bitlinear_api")


def test_cpp_bitlinear_pair(gpu, tmp_path):
    """The reference's InferenceEngine::bitlinear pair (absmax_reduce_gpu, then
    fused_sparse_bitlinear_gpu; src/inference.cu:106-117) compiled in a C++
    host program against this build's mirror headers, on the 6912x2560 FFN
    shape in fp16 and bf16: output bits equal the oracle's."""
    from spbitnet_amd import weights as W
    assert os.path.exists(BITLINEAR_EXE), "tests/cpp/bitlinear_api is not built"
    rows, cols = 6912, 2560
    L = W.random_layer(rows, cols, W.seed_for("cpp-bitlinear", rows, cols))
    a = W.normal_f32(W.seed_for("cpp-bitlinear-x", cols), cols)
    L.meta.astype("<u4").tofile(tmp_path / "meta.bin")
    L.values.astype("<u4").tofile(tmp_path / "values.bin")
    x16 = a.astype(np.float16)
    xb = O.to_bf16_bits(a)
    x16.view(np.uint16).tofile(tmp_path / "x_f16.bin")
    xb.tofile(tmp_path / "x_bf16.bin")
    print("running the C++ bitlinear program", flush=True)
    r = subprocess.run([BITLINEAR_EXE, str(tmp_path), str(rows), str(cols), str(L.meta_stride),
                        str(L.values_stride), repr(float(L.gamma))],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    for tag, xf, to_bits in (("f16", x16.astype(np.float32), O.to_f16_bits),
                             ("bf16", O.bf16_bits_to_f32(xb), O.to_bf16_bits)):
        want, _ = O.fused_bitlinear(L.meta, L.values, xf, O.absmax(xf), L.gamma, rows, cols)
        got = np.fromfile(tmp_path / f"out_{tag}.bin", dtype=np.uint16)
        assert got.size == rows
        assert (got == to_bits(want)).all(), tag
