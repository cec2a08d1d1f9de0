"""Writes the oracle's greedy tokens for the 2.4B-parameter BitNet-b1.58-2B-4T
shape (random init, Model.random(ModelConfig.bitnet_b158_2b4t(), seed=2025),
the model bench.py decodes), for the GPU tests and bench.py to compare with:

  config3      BOS + 32 seeded ids (numpy default_rng(2025)), 128 greedy steps
  config4_bs1  BOS + 2047 seeded ids (default_rng(2025)), 4096-position cache,
               32 greedy steps

The weights come from the library's device generator, so this runs on a GPU
box: the model is generated there, copied to the host, and the CPU oracle
(oracle/spb_engine_oracle.c, OpenMP over rows and attention splits) runs the
reference's generate loop (src/main.cpp:133-155) one token at a time.
usage: python tests/golden/make_decode_golden.py OUT.json
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

CASES = [("config3", 33, 128, 256), ("config4_bs1", 2048, 32, 4096)]
SEED = 2025


def prompt_of(cfg, n, seed):
    return [cfg.bos_token_id] + [int(t) for t in np.random.default_rng(seed).integers(
        0, cfg.vocab_size, n - 1)]


def main(out_path):
    import torch
    from oracle import oracle as O
    from spbitnet_amd.model import Model, ModelConfig
    cfg = ModelConfig.bitnet_b158_2b4t()
    print("generating the model on the device", flush=True)
    model = Model.random(cfg, seed=SEED)
    torch.cuda.synchronize()
    host = model.to_host()
    del model
    out = {"model": "Model.random(ModelConfig.bitnet_b158_2b4t(), seed=2025)",
           "prompt": "BOS + numpy default_rng(2025).integers(0, vocab, prompt_len - 1)"}
    for key, plen, n_new, max_seq in CASES:
        prompt = prompt_of(cfg, plen, SEED)
        ora = O.EngineOracle(host, max_seq)
        t0 = time.time()
        for i, t in enumerate(prompt[:-1]):
            ora.prefill(t)
            if i % 256 == 0:
                print(f"{key}: prefill {i}/{plen - 1} ({time.time() - t0:.0f} s)", flush=True)
        tok, toks = prompt[-1], []
        for i in range(n_new):
            tok, _ = ora.step(tok)
            toks.append(tok)
            if i % 16 == 0:
                print(f"{key}: step {i}/{n_new} ({time.time() - t0:.0f} s)", flush=True)
        out[key] = {"prompt_len": plen, "max_seq": max_seq, "tokens": toks}
        print(f"{key}: {toks[:8]} ... ({time.time() - t0:.0f} s)", flush=True)
    with open(out_path, "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main(sys.argv[1])
