"""GPU parity of the decode engine (spb_engine_*) and the device weight
generator against the CPU oracle (oracle/spb_engine_oracle.c): logits bit
for bit and greedy token ids exactly, the bar of the reference's own
generate loop (src/main.cpp:133-155) on random-init weights."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spbitnet_amd import weights as W

pytestmark = pytest.mark.gpu


def _small_config(**kw):
    from spbitnet_amd.model import ModelConfig
    base = dict(hidden_size=512, num_hidden_layers=2, num_attention_heads=8,
                num_key_value_heads=2, intermediate_size=1536, vocab_size=4096,
                max_position_embeddings=1024, head_dim=64, rms_norm_eps=1e-5,
                rope_theta=500000.0, bos_token_id=1, eos_token_id=2)
    base.update(kw)
    return ModelConfig(**base)


def _last_logits(eng):
    """The device logits of the engine's last step (a copy)."""
    import ctypes
    from spbitnet_amd import _lib
    lp = ctypes.c_void_p()
    _lib.check(eng._L.spb_engine_buffers(eng._h, ctypes.byref(lp), None), "spb_engine_buffers")
    out = torch.empty(eng._logits.numel(), dtype=torch.float32, device=eng._logits.device)
    torch.cuda.synchronize()
    _lib.memcpy_d2d(out.data_ptr(), lp.value, out.numel() * 4, None)
    torch.cuda.synchronize()
    return out


def _prompt(n, vocab, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


def test_generator_matches_host_packing(gpu):
    from spbitnet_amd import _lib
    L = _lib.load()
    for rows, cols, seed in [(64, 256, 1), (33, 640, 2), (7, 64, 3)]:
        ms, vs = cols // 32, cols // 64
        meta = torch.empty((rows, ms), dtype=torch.int32, device="cuda")
        values = torch.empty((rows, vs), dtype=torch.int32, device="cuda")
        gamma = torch.zeros(1, dtype=torch.float32, device="cuda")
        latent = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
        print(f"generator rows={rows} cols={cols}", flush=True)
        _lib.check(L.spb_generate_sparse_ternary(seed, rows, cols, meta.data_ptr(),
                                                 values.data_ptr(), ms, vs, gamma.data_ptr(),
                                                 latent.data_ptr(), None), "generate")
        torch.cuda.synchronize()
        w = latent.cpu().numpy()
        assert np.isfinite(w).all() and 0.6 < np.abs(w).mean() < 1.0
        want = W.make_layer_from_latent(w)
        assert np.array_equal(meta.cpu().numpy().view(np.uint32), want.meta)
        assert np.array_equal(values.cpu().numpy().view(np.uint32), want.values)
        g = float(gamma.item())
        assert abs(g - O.absmean(w)) <= 1e-6 * O.absmean(w)


@pytest.mark.parametrize("rows,cols,seed", [(6912, 2560, 11), (2560, 6912, 12), (33, 640, 13),
                                            (1, 64, 14)])
def test_generator_matches_host(gpu, rows, cols, seed):
    """The device generator equals its host restatement (oracle/spb_gen.c) bit
    for bit: every latent value, the packed words and the gamma bits."""
    from spbitnet_amd import _lib
    L = _lib.load()
    ms, vs = cols // 32, cols // 64
    meta = torch.empty((rows, ms), dtype=torch.int32, device="cuda")
    values = torch.empty((rows, vs), dtype=torch.int32, device="cuda")
    gamma = torch.zeros(1, dtype=torch.float32, device="cuda")
    latent = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    print(f"generator vs host rows={rows} cols={cols}", flush=True)
    _lib.check(L.spb_generate_sparse_ternary(seed, rows, cols, meta.data_ptr(), values.data_ptr(),
                                             ms, vs, gamma.data_ptr(), latent.data_ptr(), None),
               "generate")
    torch.cuda.synchronize()
    assert np.array_equal(latent.cpu().numpy().view(np.uint32).ravel(),
                          O.gen_normals(seed, rows * cols).view(np.uint32))
    hm, hv, hg = O.gen_sparse_ternary(seed, rows, cols)
    assert np.array_equal(meta.cpu().numpy().view(np.uint32), hm)
    assert np.array_equal(values.cpu().numpy().view(np.uint32), hv)
    assert np.float32(gamma.item()).view(np.uint32) == np.float32(hg).view(np.uint32)


def test_random_model_matches_host_model(gpu):
    """Model.random at the 2.4B shape (the model of the golden decode tokens)
    equals oracle.host_random_model: layers 0 and 29 word for word with their
    gamma bits, and the whole bf16 embedding / LM head."""
    from spbitnet_amd.model import Model, ModelConfig
    cfg = ModelConfig.bitnet_b158_2b4t()
    print("Model.random 2.4B vs host generator", flush=True)
    model = Model.random(cfg, seed=2025)
    torch.cuda.synchronize()
    from spbitnet_amd.weights import seed_for
    for li in (0, cfg.num_hidden_layers - 1):
        for name in O.EngineOracle.PROJ:
            s = getattr(model.layers[li], name)
            hm, hv, hg = O.gen_sparse_ternary(seed_for("model", 2025, li, name), s.rows, s.cols)
            assert np.array_equal(s.meta.cpu().numpy().view(np.uint32), hm), (li, name)
            assert np.array_equal(s.values.cpu().numpy().view(np.uint32), hv), (li, name)
            assert np.float32(s.gamma).view(np.uint32) == np.float32(hg).view(np.uint32)
    emb = model.embed_tokens.view(torch.int16).cpu().numpy().view(np.uint16).ravel()
    want = O.gen_normal_bf16(seed_for("model", 2025, "embed"), emb.size, 0.02)
    assert np.array_equal(emb, want)
    del model
    torch.cuda.empty_cache()


def _engine_pair(cfg, seed, max_seq, **kw):
    from spbitnet_amd.model import InferenceEngine, Model
    model = Model.random(cfg, seed=seed, **kw)
    torch.cuda.synchronize()
    eng = InferenceEngine(model, max_seq=max_seq)
    ora = O.EngineOracle(model.to_host(), max_seq)
    return model, eng, ora


def test_engine_forward_logits_bit_exact(gpu):
    cfg = _small_config()
    model, eng, ora = _engine_pair(cfg, seed=11, max_seq=128)
    for i, t in enumerate(_prompt(24, cfg.vocab_size, 5)):
        print(f"forward step {i}", flush=True)
        got = eng.forward(t).cpu().numpy()
        want_tok, want = ora.step(t)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            f"step {i}: max |diff| {np.abs(got - want).max()}"
        assert int(np.argmax(got)) == want_tok
    assert eng.seq_len() == 24
    eng.reset()
    ora.reset()
    got = eng.forward(7).cpu().numpy()
    assert np.array_equal(got, ora.step(7)[1])
    eng.close()


def test_engine_tied_and_dominant_inputs(gpu):
    """Embedding rows whose elements all have the same magnitude (every
    element ties for the absmax of layer 0's q/k/v prologue) and rows with
    one dominant element: logits bit-identical to the oracle on every step of
    the decode engine, and the batched engine's tokens equal the oracle's."""
    from spbitnet_amd.model import BatchInferenceEngine, InferenceEngine, Model
    cfg = _small_config()
    model = Model.random(cfg, seed=61)
    H = cfg.hidden_size
    emb = model.embed_tokens
    for t in range(8):  # |x| all equal: every product ties
        row = torch.full((H,), 0.5, dtype=torch.float32)
        row[1::2] = -0.5
        emb[t] = row.to(torch.bfloat16).to(emb.device)
    for t in range(8, 16):  # one dominant element, the rest small and distinct
        row = torch.linspace(-0.01, 0.01, H)
        row[(t * 37) % H] = 1.5 if t % 2 else -1.5
        emb[t] = row.to(torch.bfloat16).to(emb.device)
    torch.cuda.synchronize()
    eng = InferenceEngine(model, max_seq=64)
    ora = O.EngineOracle(model.to_host(), 64)
    toks = [3, 9, 0, 12, 7, 15, 1, 8, 5, 14, 2, 11]
    for i, t in enumerate(toks):
        print(f"shortcut step {i} token {t}", flush=True)
        got = eng.forward(t).cpu().numpy()
        _, want = ora.step(t)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"step {i}"
    eng.close()
    beng = BatchInferenceEngine(model, max_seq=64, batch=3)
    prompts = [toks[:4], toks[4:9], toks[9:]]
    got = beng.generate(prompts, 6, stop_at_eos=False)
    beng.close()
    host = model.to_host()
    assert got == [O.EngineOracle(host, 64).generate(p, 6) for p in prompts]


def test_engine_greedy_128_matches_oracle(gpu):
    cfg = _small_config()
    model, eng, ora = _engine_pair(cfg, seed=3, max_seq=256)
    prompt = _prompt(33, cfg.vocab_size, 9)
    print("generate 128", flush=True)
    got = eng.generate(prompt, 128, stop_at_eos=False)
    want = ora.generate(prompt, 128)
    assert len(got) == 128
    assert got == want
    # a second generation on the same engine starts from a clean state
    again = eng.generate(prompt, 16, stop_at_eos=False)
    assert again == want[:16]
    eng.close()


def test_engine_attention_splits(gpu):
    """Prompt spanning 10 of the 64-position attention splits (more than the
    combine's first batch of 4)."""
    cfg = _small_config(num_hidden_layers=1)
    model, eng, ora = _engine_pair(cfg, seed=21, max_seq=700)
    prompt = _prompt(600, cfg.vocab_size, 13)
    print("generate long", flush=True)
    got = eng.generate(prompt, 40, stop_at_eos=False)
    assert got == ora.generate(prompt, 40)
    eng.close()


def test_engine_long_context_4096(gpu):
    """Config-4 geometry on a one-layer model: a 4096-position KV cache, a
    2048-token prompt, then greedy steps past position 2048 (33 splits)."""
    cfg = _small_config(num_hidden_layers=1, max_position_embeddings=4096)
    model, eng, ora = _engine_pair(cfg, seed=23, max_seq=4096)
    prompt = _prompt(2048, cfg.vocab_size, 17)
    print("generate 2048 + 24", flush=True)
    got = eng.generate(prompt, 24, stop_at_eos=False)
    assert got == ora.generate(prompt, 24)
    eng.close()


def test_engine_split_combine_logits(gpu):
    """Steps on both sides of the 8-split boundary (position 512), logits bit
    for bit against the oracle at every step from 500: up to 8 splits the o
    projection's prologue folds them, past that attn_combine_kernel does
    (GQA groups 1, 4 and 8 at head_dim 64, 4 and 8 at head_dim 128)."""
    for nh, nkv, hd in [(8, 2, 64), (8, 8, 64), (8, 1, 64), (4, 1, 128), (8, 1, 128)]:
        cfg = _small_config(num_hidden_layers=1, hidden_size=nh * hd, num_attention_heads=nh,
                            num_key_value_heads=nkv, head_dim=hd, max_position_embeddings=1024)
        print(f"split combine nh={nh} nkv={nkv} hd={hd}", flush=True)
        model, eng, ora = _engine_pair(cfg, seed=71 + nkv + hd, max_seq=1024)
        for i, t in enumerate(_prompt(600, cfg.vocab_size, 3 + nkv)):
            got = eng.forward(t)
            want_tok, want = ora.step(t)
            if i >= 500:
                got = got.cpu().numpy()
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                    f"nh={nh} nkv={nkv} hd={hd} step {i}: max |diff| {np.abs(got - want).max()}"
                assert int(np.argmax(got)) == want_tok
        eng.close()


def test_engine_long_context_gqa_groups(gpu):
    """Past 4 splits the o projection's prologue loads the remaining splits in
    groups: GQA groups 1, 2 and 8 with head_dim 64 and group 4 with head_dim
    128, greedy steps at positions 300-315 (5 splits) against the oracle."""
    for nh, nkv, hd in [(8, 8, 64), (8, 4, 64), (8, 1, 64), (4, 1, 128)]:
        cfg = _small_config(num_hidden_layers=1, hidden_size=nh * hd, num_attention_heads=nh,
                            num_key_value_heads=nkv, head_dim=hd, max_position_embeddings=512)
        print(f"long context nh={nh} nkv={nkv} hd={hd}", flush=True)
        model, eng, ora = _engine_pair(cfg, seed=51 + nkv + hd, max_seq=320)
        prompt = _prompt(300, cfg.vocab_size, nkv + hd)
        assert eng.generate(prompt, 16, stop_at_eos=False) == ora.generate(prompt, 16)
        eng.close()


def test_engine_batched_prefill_matches_stepwise(gpu):
    """Batched prefill (per-token producers and sinks around the matrix-core
    GEMM, the prefill form of the attention kernel) against one decode step
    per prompt token on the same engine: the logits of the first generated
    step are bit-identical and the generated tokens equal; prompts that span
    several prefill passes and attention splits, GQA groups 8, 4 and 1, head
    dims 64 and 128, with and without sub-norms."""
    # 2100 tokens: three prefill passes (1024, 1024, 51 tokens) and 33 splits
    hd128 = dict(head_dim=128, hidden_size=1024)
    cases = [({}, dict(), 2, 2200, 2100), ({}, dict(sub_norms=False), 2, 96, 40),
             ({}, dict(), 8, 320, 300), ({}, dict(), 1, 64, 17), (hd128, dict(), 2, 200, 150),
             (hd128, dict(), 1, 160, 130), (hd128, dict(), 8, 96, 70)]
    for ckw, kw, nkv, max_seq, n_prompt in cases:
        cfg = _small_config(num_key_value_heads=nkv, max_position_embeddings=max(max_seq, 1024),
                            num_hidden_layers=1 if n_prompt > 1000 else 2, **ckw)
        print(f"prefill {ckw} {kw} nkv={nkv} max_seq={max_seq} prompt={n_prompt}", flush=True)
        model, eng, ora = _engine_pair(cfg, seed=61 + nkv + n_prompt, max_seq=max_seq, **kw)
        prompt = _prompt(n_prompt, cfg.vocab_size, 5 + nkv)
        eng.set_prefill_batch(16)
        got = eng.generate(prompt, 12, stop_at_eos=False)
        eng.set_prefill_batch(0)
        want = eng.generate(prompt, 12, stop_at_eos=False)
        assert got == want
        eng.set_prefill_batch(16)
        eng.generate(prompt, 1, stop_at_eos=False)
        lb = _last_logits(eng)
        eng.set_prefill_batch(0)
        eng.generate(prompt, 1, stop_at_eos=False)
        ls = _last_logits(eng)
        assert torch.equal(lb.view(torch.int32), ls.view(torch.int32))
        assert got == ora.generate(prompt, 12)
        eng.close()


def test_engine_without_sub_norms_and_gqa_variants(gpu):
    for kw, nkv in [(dict(sub_norms=False), 2), ({}, 8), ({}, 4), ({}, 1)]:
        cfg = _small_config(num_key_value_heads=nkv)
        print(f"variant {kw} nkv={nkv}", flush=True)
        model, eng, ora = _engine_pair(cfg, seed=31 + nkv, max_seq=96, **kw)
        prompt = _prompt(9, cfg.vocab_size, nkv)
        assert eng.generate(prompt, 40, stop_at_eos=False) == ora.generate(prompt, 40)
        eng.close()


def test_engine_stops_at_eos(gpu):
    cfg = _small_config(num_hidden_layers=1)
    model, eng, ora = _engine_pair(cfg, seed=41, max_seq=128)
    prompt = _prompt(5, cfg.vocab_size, 1)
    free = ora.generate(prompt, 30)
    eos = free[11]
    first = free.index(eos)
    eng.close()
    from spbitnet_amd.model import InferenceEngine
    cfg2 = _small_config(num_hidden_layers=1, eos_token_id=eos)
    model.config = cfg2
    eng = InferenceEngine(model, max_seq=128)
    got = eng.generate(prompt, 30, stop_at_eos=True)
    assert got == free[:first + 1]
    eng.close()


def test_engine_rejects_bad_input(gpu):
    from spbitnet_amd import _lib
    cfg = _small_config(num_hidden_layers=1)
    model, eng, ora = _engine_pair(cfg, seed=5, max_seq=16)
    with pytest.raises(_lib.SpbError):
        eng.forward(cfg.vocab_size)
    with pytest.raises(_lib.SpbError):
        eng.generate([1, 2, 3], 20)  # exceeds max_seq
    eng.close()


def test_engine_bitnet_2b4t_shape(gpu):
    """Full config-3 shape: first decode steps bit-exact against the oracle."""
    from spbitnet_amd.model import ModelConfig
    cfg = ModelConfig.bitnet_b158_2b4t(max_position_embeddings=4096)
    print("generating the 2.4B-parameter random model", flush=True)
    model, eng, ora = _engine_pair(cfg, seed=2025, max_seq=64)
    for i, t in enumerate(_prompt(3, cfg.vocab_size, 2025)):
        print(f"config3 step {i}", flush=True)
        got = eng.forward(t).cpu().numpy()
        want_tok, want = ora.step(t)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            f"step {i}: max |diff| {np.abs(got - want).max()}"
    eng.close()


def test_engine_forward_after_generate_at_eos(gpu):
    """generate() stopping at EOS leaves its generate-mode state (done, the
    prompt length, the EOS stop) on the device; a later forward() continues
    at the position generate reached, in forward mode, with logits equal to
    the oracle's after the same tokens."""
    from spbitnet_amd.model import InferenceEngine
    cfg = _small_config(num_hidden_layers=1)
    model, eng, ora = _engine_pair(cfg, seed=43, max_seq=128)
    prompt = _prompt(6, cfg.vocab_size, 2)
    free = ora.generate(prompt, 24)
    eos = free[9]
    eng.close()
    model.config = _small_config(num_hidden_layers=1, eos_token_id=eos)
    eng = InferenceEngine(model, max_seq=128)
    got = eng.generate(prompt, 24, stop_at_eos=True)
    want = ora.generate(prompt, 24, eos=eos)
    assert got == want and got[-1] == eos
    assert eng.seq_len() == len(prompt) - 1 + len(got)
    for i, t in enumerate([eos, 17, eos, 3]):
        print(f"forward after generate {i}", flush=True)
        g = eng.forward(t).cpu().numpy()
        wt, w = ora.step(t)
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"step {i}"
    assert eng.seq_len() == len(prompt) - 1 + len(got) + 4
    eng.close()


def test_engine_decode_steps_then_forward(gpu):
    """decode_steps() advances the device position without a host sync;
    seq_len() reads it back and forward() continues there."""
    cfg = _small_config(num_hidden_layers=1)
    model, eng, ora = _engine_pair(cfg, seed=47, max_seq=128)
    prompt = _prompt(7, cfg.vocab_size, 3)
    assert eng.generate(prompt, 0, stop_at_eos=False) == []
    assert eng.seq_len() == len(prompt) - 1
    eng.decode_steps(5)
    assert eng.seq_len() == len(prompt) - 1 + 5
    want = ora.generate(prompt, 5)
    g = eng.forward(want[-1]).cpu().numpy()
    wt, w = ora.step(want[-1])
    assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
    eng.close()


def test_engine_rejects_short_strides(gpu):
    """spb_engine_create checks that every projection's strides cover a row
    before anything is launched (an understated stride would make the
    projection kernels read past each row)."""
    from spbitnet_amd import _lib
    from spbitnet_amd.model import InferenceEngine, Model
    cfg = _small_config(num_hidden_layers=1)
    model = Model.random(cfg, seed=5)
    q = model.layers[0].q_proj
    q.meta_stride, keep = 4, q.meta_stride  # cols 512 need 16 meta words per row
    with pytest.raises(_lib.SpbError, match="q_proj"):
        InferenceEngine(model, max_seq=16)
    q.meta_stride = keep
    d = model.layers[0].down_proj
    d.values_stride, keep = 2, d.values_stride
    with pytest.raises(_lib.SpbError, match="down_proj"):
        InferenceEngine(model, max_seq=16)
    d.values_stride = keep
    InferenceEngine(model, max_seq=16).close()


GOLDEN_2B4T = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                           "decode_2b4t_tokens.json")


def test_engine_bitnet_2b4t_greedy_128_golden(gpu):
    """Config 3 at full shape: BOS + 32 seeded ids, then 128 greedy steps on
    the 2.4B-parameter model, tokens equal to the oracle's (committed by
    tests/golden/make_decode_golden.py from the same device-generated
    weights; the first 4 are recomputed here by the oracle live)."""
    import json
    from spbitnet_amd.model import InferenceEngine, Model, ModelConfig
    gold = json.load(open(GOLDEN_2B4T))
    cfg = ModelConfig.bitnet_b158_2b4t()
    print("generating the 2.4B-parameter random model", flush=True)
    model = Model.random(cfg, seed=2025)
    prompt = [cfg.bos_token_id] + _prompt(32, cfg.vocab_size, 2025)
    eng = InferenceEngine(model, max_seq=256)
    print("generate 128", flush=True)
    got = eng.generate(prompt, 128, stop_at_eos=False)
    assert got == gold["config3"]["tokens"]
    eng.close()
    print("oracle: 4 live steps", flush=True)
    assert O.EngineOracle(model.to_host(), 64).generate(prompt, 4) == got[:4]


def _bench_prompt(cfg, n, seed):
    """bench.py's prompts: BOS + n - 1 ids from numpy default_rng(seed)."""
    return [cfg.bos_token_id] + _prompt(n - 1, cfg.vocab_size, seed)


def test_engine_bitnet_2b4t_config4_bs1_golden(gpu):
    """Config 4 at full shape and batch 1: the 2.4B-parameter model, a
    2048-token prompt into a 4096-position cache (the batched prefill), then
    128 greedy steps past position 2048 (33-35 attention splits, the
    separate split-combine kernel), tokens equal to the oracle's (committed
    by tests/golden/make_decode_golden.py on the host-generated copy of the
    same weights)."""
    import json
    from spbitnet_amd.model import InferenceEngine, Model, ModelConfig
    gold = json.load(open(GOLDEN_2B4T))["config4_bs1"]
    cfg = ModelConfig.bitnet_b158_2b4t()
    print("generating the 2.4B-parameter random model", flush=True)
    model = Model.random(cfg, seed=2025)
    prompt = _bench_prompt(cfg, gold["prompt_len"], gold["prompt_seed"])
    assert len(prompt) == 2048 and len(gold["tokens"]) == 128
    eng = InferenceEngine(model, max_seq=gold["max_seq"])
    print("config 4 bs=1: prefill + 128 steps", flush=True)
    assert eng.generate(prompt, 128, stop_at_eos=False) == gold["tokens"]
    eng.close()


def test_batch_engine_bitnet_2b4t_config4_b32_golden(gpu):
    """Config 4 at full shape and batch 32: bench.py's 32 prompts of 2048
    tokens (sequence 0 from seed 2025, sequence b from seed 4000 + b) in
    4096-position caches, 128 greedy steps on the batched engine.  Every
    sequence with committed oracle tokens (0, 7, 17 and 31) equals them for
    all 128 steps; four more sequences equal the bs=1
    engine's generate; and sequence 0's logits of the last step match the bs=1
    engine's (argmax row bit for bit, every row within 1e-3 of the largest)."""
    import json
    from spbitnet_amd.model import BatchInferenceEngine, InferenceEngine, Model, ModelConfig
    gold = json.load(open(GOLDEN_2B4T))
    slots = {0: gold["config4_bs1"]}
    for b in (7, 17, 31):
        g = gold.get(f"config4_seq{4000 + b}")
        if g is not None:
            slots[b] = g
    assert len(slots) == 4
    cfg = ModelConfig.bitnet_b158_2b4t()
    print("generating the 2.4B-parameter random model", flush=True)
    model = Model.random(cfg, seed=2025)
    prompts = [_bench_prompt(cfg, 2048, 2025 if b == 0 else 4000 + b) for b in range(32)]
    beng = BatchInferenceEngine(model, max_seq=4096, batch=32)
    print("batch 32: prefill + 128 steps", flush=True)
    got = beng.generate(prompts, 128, stop_at_eos=False)
    blog = beng.last_logits()[0].cpu().numpy()
    beng.close()
    torch.cuda.empty_cache()
    for b, g in slots.items():
        assert got[b] == g["tokens"], f"sequence {b}"
    eng = InferenceEngine(model, max_seq=4096)
    print("bs=1 engine: sequences 0, 5, 12, 24, 30", flush=True)
    for b in (5, 12, 24, 30):
        assert eng.generate(prompts[b], 128, stop_at_eos=False) == got[b], f"sequence {b}"
    eng.generate(prompts[0], 127, stop_at_eos=False)
    one = eng.forward(got[0][126]).cpu().numpy()
    eng.close()
    tok = got[0][127]
    assert int(np.argmax(one)) == tok
    assert blog[tok].view(np.uint32) == one[tok].view(np.uint32)
    assert np.abs(blog - one).max() <= 1e-3 * np.abs(one).max()


def test_full_width_long_context(gpu):
    """Config-4 geometry at full width (hidden 2560, 20/5 heads, FFN 6912,
    vocab 128256) on a 2-layer model: a 2048-token prompt into a
    4096-position cache, 24 greedy steps, on the bs=1 engine and, for that
    prompt and a 1500-token one together, on the batched engine; tokens
    equal to the oracle's."""
    from spbitnet_amd.model import BatchInferenceEngine, InferenceEngine, Model, ModelConfig
    cfg = ModelConfig.bitnet_b158_2b4t()
    cfg.num_hidden_layers = 2
    print("generating the 2-layer full-width model", flush=True)
    model = Model.random(cfg, seed=77)
    p0 = [cfg.bos_token_id] + _prompt(2047, cfg.vocab_size, 5)
    p1 = [cfg.bos_token_id] + _prompt(1499, cfg.vocab_size, 6)
    eng = InferenceEngine(model, max_seq=4096)
    got0 = eng.generate(p0, 24, stop_at_eos=False)
    eng.close()
    beng = BatchInferenceEngine(model, max_seq=4096, batch=2)
    got = beng.generate([p0, p1], 24, stop_at_eos=False)
    beng.close()
    print("oracle (2 sequences)", flush=True)
    host = model.to_host()
    import concurrent.futures
    with concurrent.futures.ThreadPoolExecutor(2) as pool:
        want = list(pool.map(lambda p: O.EngineOracle(host, 4096).generate(p, 24), [p0, p1]))
    assert got0 == want[0]
    assert got == want


def test_engine_decode_step_runs_cross_buckets(gpu):
    """decode_steps() replays one token-step graph per step, each chosen by the
    bucket of its own position: runs that cross a 256-position bucket edge,
    and the 512-position edge where the split combine moves out of the o
    projection, leave the same tokens and logits as the oracle's one step at
    a time."""
    cfg = _small_config(num_hidden_layers=2)
    model, eng, ora = _engine_pair(cfg, seed=53, max_seq=1024)
    for plen, steps in ((250, 11), (507, 10)):
        prompt = _prompt(plen, cfg.vocab_size, plen)
        assert eng.generate(prompt, 0, stop_at_eos=False) == []
        eng.decode_steps(steps)
        assert eng.seq_len() == len(prompt) - 1 + steps
        want = ora.generate(prompt, steps)
        g = eng.forward(want[-1]).cpu().numpy()
        wt, w = ora.step(want[-1])
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), plen
        got = eng.generate(prompt, steps, stop_at_eos=False)
        assert got == want[:steps], plen
    eng.close()
