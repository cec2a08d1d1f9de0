"""Writes the oracle's greedy tokens for the 2.4B-parameter BitNet-b1.58-2B-4T
shape (random init, Model.random(ModelConfig.bitnet_b158_2b4t(), seed=2025),
the model bench.py decodes), for the GPU tests and bench.py to compare with:

  config3          BOS + 32 ids from numpy default_rng(2025), 256-position
                   cache, 128 greedy steps
  config4_bs1      BOS + 2047 ids from default_rng(2025), 4096-position cache,
                   128 greedy steps (sequence 0 of bench.py's batches)
  config4_seq4007  BOS + 2047 ids from default_rng(4007): sequence 7 of the
  config4_seq4017  batch-8 and batch-32 prompt sets (4017: sequence 17 and
  config4_seq4031  4031: sequence 31 of the batch-32 set), 4096-position
                   cache, 128 greedy steps each

No GPU is needed: the model comes from the host restatement of the library's
generator (oracle.host_random_model, oracle/spb_gen.c), which reproduces the
device's weights bit for bit (tests/test_gpu_engine.py checks that on the
GPU), and the CPU oracle (oracle/spb_engine_oracle.c, OpenMP over rows and
attention splits) runs the reference's generate loop (src/main.cpp:133-155)
one token at a time.  The file is rewritten after every case.
usage: python tests/golden/make_decode_golden.py OUT.json [case ...]
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

# key, prompt seed, prompt length, generated tokens, cache positions
CASES = [("config3", 2025, 33, 128, 256), ("config4_bs1", 2025, 2048, 128, 4096),
         ("config4_seq4017", 4017, 2048, 128, 4096), ("config4_seq4031", 4031, 2048, 128, 4096),
         ("config4_seq4007", 4007, 2048, 128, 4096)]
SEED = 2025


def prompt_of(cfg, n, seed):
    return [cfg.bos_token_id] + [int(t) for t in np.random.default_rng(seed).integers(
        0, cfg.vocab_size, n - 1)]


def main(out_path, only=()):
    from oracle import oracle as O
    from spbitnet_amd.model import ModelConfig
    cfg = ModelConfig.bitnet_b158_2b4t()
    t0 = time.time()
    print("generating the model on the host", flush=True)
    host = O.host_random_model(cfg, seed=SEED)
    print(f"model ready ({time.time() - t0:.0f} s)", flush=True)
    out = {"model": "Model.random(ModelConfig.bitnet_b158_2b4t(), seed=2025)",
           "prompt": "BOS + numpy default_rng(prompt_seed).integers(0, vocab, prompt_len - 1)"}
    if os.path.exists(out_path):
        with open(out_path) as f:
            old = json.load(f)
        out.update({k: v for k, v in old.items() if isinstance(v, dict)})
    for key, pseed, plen, n_new, max_seq in CASES:
        if only and key not in only:
            continue
        prompt = prompt_of(cfg, plen, pseed)
        ora = O.EngineOracle(host, max_seq)
        t1 = time.time()
        for i, t in enumerate(prompt[:-1]):
            ora.prefill(t)
            if i % 256 == 0:
                print(f"{key}: prefill {i}/{plen - 1} ({time.time() - t1:.0f} s)", flush=True)
        tok, toks = prompt[-1], []
        for i in range(n_new):
            tok, _ = ora.step(tok)
            toks.append(tok)
            if i % 16 == 0:
                print(f"{key}: step {i}/{n_new} ({time.time() - t1:.0f} s)", flush=True)
        out[key] = {"prompt_seed": pseed, "prompt_len": plen, "max_seq": max_seq, "tokens": toks}
        print(f"{key}: {toks[:8]} ... ({time.time() - t1:.0f} s)", flush=True)
        del ora
        with open(out_path + ".tmp", "w") as f:
            json.dump(out, f, indent=1)
        os.replace(out_path + ".tmp", out_path)


if __name__ == "__main__":
    main(sys.argv[1], tuple(sys.argv[2:]))
