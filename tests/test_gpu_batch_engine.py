"""GPU parity of the batched decode engine (spb_batch_engine_*, BASELINE
config 4 at batch 8 and 32): every sequence of a batch, with distinct ragged
prompts, produces exactly the greedy tokens the CPU oracle's single-sequence
generate (src/main.cpp:133-155 per sequence, oracle/spb_engine_oracle.c)
produces for it, and those of the bs=1 engine."""
import concurrent.futures
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    from spbitnet_amd.model import ModelConfig
    base = dict(hidden_size=512, num_hidden_layers=2, num_attention_heads=8,
                num_key_value_heads=2, intermediate_size=1536, vocab_size=4096,
                max_position_embeddings=4096, head_dim=64, rms_norm_eps=1e-5,
                rope_theta=500000.0, bos_token_id=1, eos_token_id=2)
    base.update(kw)
    return ModelConfig(**base)


def _prompts(n, vocab, lo, hi, seed):
    rng = np.random.default_rng(seed)
    return [[int(t) for t in rng.integers(0, vocab, int(rng.integers(lo, hi + 1)))]
            for _ in range(n)]


def _oracle_tokens(host, max_seq, prompts, n_new, eos=-1):
    """The oracle's single-sequence generate for each prompt (host threads,
    one oracle engine per sequence)."""
    def one(p):
        return O.EngineOracle(host, max_seq).generate(p, n_new, eos)
    workers = min(16, os.cpu_count() or 1, len(prompts))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        return list(pool.map(one, prompts))


@pytest.mark.parametrize("batch", [8, 17, 25, 32])
def test_batch_decode_matches_oracle(gpu, batch):
    """Ragged prompts of 260-700 tokens (5-11 of the 64-position attention
    splits) in a 4096-position cache, 16 greedy steps per sequence.  17
    sequences: the GEMM's 32-token tile with 15 padding tokens (masked in
    the sink epilogue) and LM-head groups of 8, 8 and 1.  25 and 32
    sequences: the layers step in two groups of sequences (12 + 13, 16 + 16)
    on parallel branches of the step graph, joined for the LM head."""
    from spbitnet_amd.model import BatchInferenceEngine, InferenceEngine, Model
    cfg = _cfg()
    model = Model.random(cfg, seed=101 + batch)
    torch.cuda.synchronize()
    prompts = _prompts(batch, cfg.vocab_size, 260, 700, seed=batch)
    print(f"batch {batch}: batched generate", flush=True)
    eng = BatchInferenceEngine(model, max_seq=4096, batch=batch)
    got = eng.generate(prompts, 16, stop_at_eos=False)
    assert [len(g) for g in got] == [16] * batch
    print(f"batch {batch}: oracle", flush=True)
    want = _oracle_tokens(model.to_host(), 4096, prompts, 16)
    for b in range(batch):
        assert got[b] == want[b], f"sequence {b} (prompt {len(prompts[b])})"
    # a second generation on the same engine with fewer sequences than slots
    print(f"batch {batch}: partial batch", flush=True)
    again = eng.generate(prompts[: batch // 2], 8, stop_at_eos=False)
    assert again == [w[:8] for w in want[: batch // 2]]
    eng.close()
    # the bs=1 engine agrees on a few sequences
    one = InferenceEngine(model, max_seq=4096)
    for b in (0, batch - 1):
        assert one.generate(prompts[b], 16, stop_at_eos=False) == want[b]
    one.close()


def test_batch_decode_gqa_variants_and_eos(gpu):
    """GQA groups 1, 4 and 8 with head_dim 64 and 128, models without
    sub-norms, short prompts (one-token prompts included), and EOS stops
    that end some sequences before others."""
    from spbitnet_amd.model import BatchInferenceEngine, Model
    cases = [(dict(num_key_value_heads=8), {}), (dict(num_key_value_heads=1), {}),
             (dict(hidden_size=512, num_attention_heads=4, num_key_value_heads=1, head_dim=128),
              dict(sub_norms=False))]
    for i, (ckw, mkw) in enumerate(cases):
        cfg = _cfg(max_position_embeddings=512, **ckw)
        print(f"batch variant {ckw} {mkw}", flush=True)
        model = Model.random(cfg, seed=201 + i, **mkw)
        prompts = _prompts(5, cfg.vocab_size, 1, 90, seed=7 + i)
        prompts[0] = prompts[0][:1]
        want = _oracle_tokens(model.to_host(), 512, prompts, 20)
        eng = BatchInferenceEngine(model, max_seq=512, batch=6)
        assert eng.generate(prompts, 20, stop_at_eos=False) == want
        eng.close()
        # EOS: the token sequence 0 generates at step 6 ends it there
        eos = want[0][6]
        model.config = _cfg(max_position_embeddings=512, eos_token_id=eos, **ckw)
        eng = BatchInferenceEngine(model, max_seq=512, batch=6)
        got = eng.generate(prompts, 20, stop_at_eos=True)
        for b in range(5):
            cut = want[b].index(eos) + 1 if eos in want[b] else 20
            assert got[b] == want[b][:cut], f"sequence {b}"
        eng.close()


def test_batch_decode_crosses_position_buckets(gpu):
    """The step graph is chosen per step by an upper bound of the largest
    live position, in buckets of 256 positions whose graphs launch the
    attention on the splits below the bucket's end only.  The longest
    prompt ends at position 249, so its steps cross from the first bucket
    into the second (split 4 starts at 256) during one generation; then a
    generation that starts in the second bucket, and one back in the first
    (the bound restarts from the new prompts)."""
    from spbitnet_amd.model import BatchInferenceEngine, Model
    cfg = _cfg(max_position_embeddings=512)
    model = Model.random(cfg, seed=417)
    host = model.to_host()
    rng = np.random.default_rng(417)
    eng = BatchInferenceEngine(model, max_seq=512, batch=4)
    for lens, n_new in (([250, 1, 244, 120], 14), ([497, 3], 10), ([30, 255], 4)):
        prompts = [[int(t) for t in rng.integers(0, cfg.vocab_size, n)] for n in lens]
        print(f"bucket crossing: prompts {lens}, {n_new} steps", flush=True)
        want = _oracle_tokens(host, 512, prompts, n_new)
        got = eng.generate(prompts, n_new, stop_at_eos=False)
        for b in range(len(lens)):
            assert got[b] == want[b], f"prompts {lens}: sequence {b}"
    eng.close()


def test_batch_decode_steps_cross_bucket(gpu):
    """decode_steps() continues a generation without a host round trip,
    choosing each step's graph from the position bound that generate()
    left: a prefill-only generate (no new tokens) of prompts ending at
    positions 246-249, then 14 decode steps that cross into the
    256-position bucket; the tokens each sequence appends to its buffer
    equal the oracle's generate."""
    from spbitnet_amd.model import BatchInferenceEngine, Model
    cfg = _cfg(max_position_embeddings=512)
    model = Model.random(cfg, seed=419)
    rng = np.random.default_rng(419)
    lens = [250, 247, 249, 248, 250, 247]
    prompts = [[int(t) for t in rng.integers(0, cfg.vocab_size, n)] for n in lens]
    want = _oracle_tokens(model.to_host(), 512, prompts, 14)
    eng = BatchInferenceEngine(model, max_seq=512, batch=6)
    assert eng.generate(prompts, 0, stop_at_eos=False) == [[] for _ in lens]
    eng.decode_steps(14)
    tok = eng.token_buffer().cpu()
    eng.close()
    for b, n in enumerate(lens):
        assert tok[b, n:n + 14].tolist() == want[b], f"sequence {b}"


@pytest.mark.parametrize("heads,kv,batch", [(8, 2, 40), (8, 1, 36), (4, 2, 48)])
def test_batch_decode_split_k_head_dim_128(gpu, heads, kv, batch):
    """At 33-64 sequences the GEMMs take the 64x32 tile (2-pair chunks), and
    intermediate 3072 makes the down projection's rows 6 chunks long, so its
    GEMM runs split over K (each part's partial tile written through to
    memory, the last block of each tile adding them and running the residual
    sink); head_dim 128 with GQA groups 4, 8 and 2 at 36-48 sequences.
    Ragged prompts (1-300 tokens, 1-5 attention splits), EOS stops that
    finish some sequences early, then a second generation with fewer
    sequences than slots; tokens equal the oracle's single-sequence
    generate."""
    from spbitnet_amd.model import BatchInferenceEngine, Model
    cfg = _cfg(hidden_size=heads * 128, num_attention_heads=heads, num_key_value_heads=kv,
               head_dim=128, intermediate_size=3072, max_position_embeddings=512)
    model = Model.random(cfg, seed=301 + heads + kv)
    host = model.to_host()
    prompts = _prompts(batch, cfg.vocab_size, 1, 300, seed=batch + heads)
    prompts[1] = prompts[1][:1]
    print(f"split-K G={heads // kv} batch {batch}: oracle", flush=True)
    want = _oracle_tokens(host, 512, prompts, 12)
    eng = BatchInferenceEngine(model, max_seq=512, batch=batch)
    got = eng.generate(prompts, 12, stop_at_eos=False)
    for b in range(batch):
        assert got[b] == want[b], f"sequence {b} (prompt {len(prompts[b])})"
    eng.close()
    # EOS: the token sequence 0 generates at step 4 ends the sequences that
    # produce it; the others run on
    eos = want[0][4]
    model.config = _cfg(hidden_size=heads * 128, num_attention_heads=heads,
                        num_key_value_heads=kv, head_dim=128, intermediate_size=3072,
                        max_position_embeddings=512, eos_token_id=eos)
    eng = BatchInferenceEngine(model, max_seq=512, batch=batch)
    got = eng.generate(prompts, 12, stop_at_eos=True)
    for b in range(batch):
        cut = want[b].index(eos) + 1 if eos in want[b] else 12
        assert got[b] == want[b][:cut], f"sequence {b}"
    again = eng.generate(prompts[: batch - 5], 6, stop_at_eos=False)
    assert again == [w[:6] for w in want[: batch - 5]]
    eng.close()


def test_batch_engine_rejects_bad_input(gpu):
    from spbitnet_amd import _lib
    from spbitnet_amd.model import BatchInferenceEngine, Model
    cfg = _cfg(num_hidden_layers=1, max_position_embeddings=64)
    model = Model.random(cfg, seed=3)
    eng = BatchInferenceEngine(model, max_seq=64, batch=4)
    with pytest.raises(_lib.SpbError):
        eng.generate([[1, 2]] * 5, 4)           # more sequences than slots
    with pytest.raises(_lib.SpbError):
        eng.generate([[1] * 60], 8)             # exceeds max_seq
    with pytest.raises(_lib.SpbError):
        eng.generate([[1], []], 4)              # empty prompt
    with pytest.raises(_lib.SpbError):
        eng.generate([[cfg.vocab_size]], 4)     # token out of range
    assert eng.generate([[5, 6, 7]], 4, stop_at_eos=False) == \
        _oracle_tokens(model.to_host(), 64, [[5, 6, 7]], 4)
    eng.close()


def test_batch_decode_odd_shapes(gpu):
    """Shapes off the 2B model's multiples: hidden 640 (the LM heads' partial
    last 512-element step), vocabulary 4093 (blocks and row octets that end
    inside a row group), GQA group 2, and 12 sequences (a last group of 4 in
    the batched LM head); tokens equal to the oracle's single-sequence
    generate on the batched and the bs=1 engine."""
    from spbitnet_amd.model import BatchInferenceEngine, InferenceEngine, Model
    cfg = _cfg(hidden_size=640, num_attention_heads=10, num_key_value_heads=5,
               intermediate_size=1664, vocab_size=4093, max_position_embeddings=512)
    model = Model.random(cfg, seed=311)
    prompts = _prompts(12, cfg.vocab_size, 1, 300, seed=19)
    print("oracle", flush=True)
    want = _oracle_tokens(model.to_host(), 512, prompts, 12)
    eng = BatchInferenceEngine(model, max_seq=512, batch=12)
    assert eng.generate(prompts, 12, stop_at_eos=False) == want
    eng.close()
    one = InferenceEngine(model, max_seq=512)
    for b in (0, 7):
        assert one.generate(prompts[b], 12, stop_at_eos=False) == want[b]
    one.close()


def _lm_bound_c(H):
    """lm_bound_c (csrc/engine.hip): the batched LM head's error-bound constant."""
    return np.float32(1.25 * (H + H // 64 + 8) * 2.0 ** -23)


@pytest.mark.parametrize("shape", ["base", "odd"])
def test_batch_lm_head_logits_within_bound(gpu, shape):
    """The batched LM head computes the logits on the bf16 matrix cores and
    recomputes exactly (the bs=1 chain) only the rows that could hold the
    maximum.  Against the oracle's logits of the same step: each sequence's
    argmax row is bit-identical, every row lies within 2 c |w| |x| (the
    bound the candidate selection relies on), the measured error is at
    least 100x inside it, and the largest error is below 1e-3 of the
    largest logit."""
    from spbitnet_amd.model import BatchInferenceEngine, Model
    if shape == "base":
        cfg, n_seq, n_new = _cfg(), 20, 5
    else:
        cfg, n_seq, n_new = _cfg(hidden_size=640, num_attention_heads=10, num_key_value_heads=5,
                                 intermediate_size=1664, vocab_size=4093,
                                 max_position_embeddings=512), 5, 4
    model = Model.random(cfg, seed=411 if shape == "base" else 412)
    torch.cuda.synchronize()
    prompts = _prompts(n_seq, cfg.vocab_size, 1, 200, seed=23)
    eng = BatchInferenceEngine(model, max_seq=512, batch=n_seq)
    got_tok = eng.generate(prompts, n_new, stop_at_eos=False)
    got = eng.last_logits().cpu().numpy()
    eng.close()
    host = model.to_host()
    W = O.bf16_bits_to_f32(host["embed"]).astype(np.float64)
    wn = np.sqrt((W * W).sum(1))
    c = float(_lm_bound_c(cfg.hidden_size))
    for b, p in enumerate(prompts):
        ora = O.EngineOracle(host, 512)
        for t in p[:-1]:
            ora.prefill(t)
        tok, toks = p[-1], []
        for _ in range(n_new):
            tok, want = ora.step(tok)
            toks.append(tok)
        assert got_tok[b] == toks, b
        xn = ora.debug("xn").astype(np.float64)
        bound = c * wn * np.sqrt((xn * xn).sum())
        err = np.abs(got[b].astype(np.float64) - want.astype(np.float64))
        assert got[b][tok].view(np.uint32) == want[tok].view(np.uint32), b
        assert (err <= 2 * bound).all(), b
        assert (err / bound).max() < 1e-2, (b, (err / bound).max())
        assert err.max() <= 1e-3 * np.abs(want).max(), b
