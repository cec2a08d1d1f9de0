"""Writes tests/golden/loader_model/: the synthetic model directory of the
reference's loader test, create_test_model (tests/test_model_loader.cu:52-191),
byte for byte in its data files: hidden 8, one layer, one (kv) head,
intermediate 16, vocab 32; every sparse row is groups of {+1, -1, 0, 0}
(bitmap 0x3, signs 0b10) with gamma 0.5; fp16 embedding of 1.0 (0x3C00);
float32 norms of 1.0; tied LM head; no sub-norms.  The JSON files hold the
same keys and values (nlohmann's dump(2) sorts keys, so they are sorted here
too).  Run from the repository root: python tests/golden/make_loader_fixture.py
"""
import json
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "loader_model")
H, V, I = 8, 32, 16


def main():
    os.makedirs(os.path.join(OUT, "weights"), exist_ok=True)
    config = {
        "model_type": "bitnet", "hidden_size": H, "num_hidden_layers": 1,
        "num_attention_heads": 1, "num_key_value_heads": 1, "intermediate_size": I,
        "vocab_size": V, "max_position_embeddings": 64, "rms_norm_eps": 1e-5,
        "rope_theta": 10000.0, "head_dim": H, "hidden_act": "relu2",
        "tie_word_embeddings": True, "bos_token_id": 0, "eos_token_id": 1,
    }
    with open(os.path.join(OUT, "config.json"), "w") as f:
        json.dump(config, f, indent=2, sort_keys=True)

    def write(rel, arr):
        arr.tofile(os.path.join(OUT, rel))

    def sparse(name, rows, cols):
        groups = cols // 4
        ms, vs = (groups + 7) // 8, (groups + 15) // 16
        meta = np.zeros((rows, ms), "<u4")
        values = np.zeros((rows, vs), "<u4")
        for g in range(groups):
            # w = {+1, -1, 0, 0}: positions 0 and 1 kept, the second negative
            meta[:, g // 8] |= np.uint32(0x3 << (4 * (g % 8)))
            values[:, g // 16] |= np.uint32(0x2 << (2 * (g % 16)))
        write(f"weights/{name}.meta", meta)
        write(f"weights/{name}.values", values)
        return {"meta_file": f"weights/{name}.meta", "values_file": f"weights/{name}.values",
                "dtype": "sparse_ternary", "shape": [rows, cols], "meta_stride": ms,
                "values_stride": vs, "gamma": 0.5, "meta_nbytes": meta.nbytes,
                "values_nbytes": values.nbytes}

    def f16_ones(name, count):
        write(f"weights/{name}.bin", np.full(count, 0x3C00, "<u2"))
        return {"file": f"weights/{name}.bin", "dtype": "float16", "nbytes": count * 2}

    def f32_ones(name, count):
        write(f"weights/{name}.bin", np.ones(count, "<f4"))
        return {"file": f"weights/{name}.bin", "dtype": "float32", "shape": [count],
                "nbytes": count * 4}

    w = {}
    e = f16_ones("embed_tokens", V * H)
    e["shape"] = [V, H]
    w["embed_tokens"] = e
    w["norm"] = f32_ones("norm", H)
    w["lm_head"] = {"tied_to": "embed_tokens", "dtype": "tied"}
    p = "layers.0"
    w[p + ".input_layernorm"] = f32_ones(p + ".input_layernorm", H)
    w[p + ".post_attention_layernorm"] = f32_ones(p + ".post_attention_layernorm", H)
    for name, rows, cols in [("self_attn.q_proj", H, H), ("self_attn.k_proj", H, H),
                             ("self_attn.v_proj", H, H), ("self_attn.o_proj", H, H),
                             ("mlp.gate_proj", I, H), ("mlp.up_proj", I, H),
                             ("mlp.down_proj", H, I)]:
        w[f"{p}.{name}"] = sparse(f"{p}.{name}", rows, cols)
    with open(os.path.join(OUT, "manifest.json"), "w") as f:
        json.dump({"format_version": 1, "weights": w}, f, indent=2, sort_keys=True)


if __name__ == "__main__":
    main()
