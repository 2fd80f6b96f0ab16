"""The north-star workloads of the 3B decoder on the GPU against the oracle.

Model: 28 layers, hidden 3072, 24/8 heads, FFN 8192, vocab 83968, N(0, 0.02)
weights with unit norm gains (the bench's model). Each test runs one workload
at its real size:

- 256-token prefill, then 400 greedy steps (KV 257 -> 656): teacher-forced
  logits against the oracle's own greedy stream, and the GPU's free-running
  greedy stream (yuear_generate_tokens, sampling.cpp:185-288) against the
  oracle's tokens. Over 28 bf16 layers the two sides differ by ~0.1 in the
  logits, so a token may differ only where the oracle's top-2 gap is within
  that difference (a near-tie); the first divergence, its gap and the share
  of logits within 2e-2 abs + 1e-2 rel are reported.
- CFG pair (512 + 512 prompt ids, scale 1.5, T 1.0, top-k 50, top-p 0.93),
  1024 sampled tokens: at every step the GPU sampler's token on the GPU's
  logits must equal the oracle's guided_logits -> distribution -> draw on the
  same logits (sampling.cpp:100-132, 244-250); a stretch of steps after the
  prefill and one step at KV 1536 are compared with the oracle run from the
  GPU's cache under the fidelity rule.
- 3000-token prefill, then device-side greedy decoding to KV 8192; the step
  at KV 8192 is compared with the oracle run from the GPU's cache.
- 8 independent sequences, prompts U[128, 2048], capacity 6144, 16 batched
  device steps, then one batched step whose every sequence is compared with
  the oracle running that sequence alone from its cache.

The fidelity rule (conftest.check_fidelity; tools/limits.py:21-79 in the
reference) bounds the GPU's distance to the fp64-accumulating oracle by twice
the fp32 oracle's own distance to it.
"""
import numpy as np
import pytest

from conftest import MODEL_3B, check_fidelity

pytestmark = pytest.mark.gpu

V = MODEL_3B["vocab_size"]
LAYERS = MODEL_3B["num_hidden_layers"]


@pytest.fixture(scope="module")
def pair(yuear_lib, oracle):
    w = yuear_lib.random_weights(MODEL_3B, 20251201)
    engine = yuear_lib.Engine(MODEL_3B, w)
    model = oracle.Model(MODEL_3B, w)
    yield engine, model, oracle
    oracle.lib().oracle_set_accumulation(0)
    engine.close()


def f32(oracle, bits):
    return oracle.bf16_to_f32(bits).astype(np.float64)


def oracle_step_from(model, oracle, kv, n, token, capacity, modes=(0, 1)):
    """Oracle logits of one step after the n cached slots kv (per layer
    (k, v)), in fp32 and fp64 accumulation."""
    out = {}
    for mode in modes:
        oracle.lib().oracle_set_accumulation(mode)
        try:
            cache = model.cache(capacity)
            for layer, (k, v) in enumerate(kv):
                cache.keys(layer)[:, :n] = k
                cache.values(layer)[:, :n] = v
            cache.offset = n
            out[mode] = model.step(token, cache)
        finally:
            oracle.lib().oracle_set_accumulation(0)
    return out


def test_cfg2_prefill_256_greedy_400(pair):
    engine, model, oracle = pair
    rng = np.random.default_rng(2002)
    prompt = rng.integers(0, V, size=256).tolist()
    n = 400
    print("[cfg2] oracle prefill 256 + 400 greedy steps", flush=True)
    cache = model.cache(256 + n)
    logits = model.prefill(prompt, cache)
    o_tokens, o_logits = [], []
    for i in range(n):
        o_logits.append(logits)
        o_tokens.append(int(np.argmax(f32(oracle, logits))))  # greedy: lowest index on ties
        if i + 1 < n:
            logits = model.step(o_tokens[-1], cache)
    print("[cfg2] GPU teacher-forced steps", flush=True)
    s = engine.session(1, 256 + n)
    g_logits = [s.prefill(0, prompt)] + [s.step(t)[0] for t in o_tokens[:-1]]
    s.close()
    within, flips = [], []
    for i, (g, o) in enumerate(zip(g_logits, o_logits)):
        gf, of = f32(oracle, g), f32(oracle, o)
        diff = np.abs(gf - of)
        within.append(np.mean(diff <= 2e-2 + 1e-2 * np.abs(of)))
        top = np.sort(of)[-2:]
        if gf.argmax() != of.argmax():
            flips.append((i, top[1] - top[0], diff.max()))
            # a different greedy token only at a near-tie the two sides'
            # own difference can explain
            assert top[1] - top[0] <= 2 * diff.max(), (i, top, diff.max())
    print("[cfg2] GPU free-running greedy stream (device sampler)", flush=True)
    greedy = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                  penalty_window=50, min_tokens=0, max_tokens=n)
    g_tokens, timing, _ = engine.generate_tokens(prompt, greedy, 0)
    assert len(g_tokens) == n
    first = next((i for i in range(n) if g_tokens[i] != o_tokens[i]), None)
    gap = None
    if first is not None:
        top = np.sort(f32(oracle, o_logits[first]))[-2:]
        gap = top[1] - top[0]
    print(f"[cfg2] logits within 2e-2 abs + 1e-2 rel: mean {np.mean(within):.4f} "
          f"min {np.min(within):.4f}; teacher-forced argmax flips {len(flips)} {flips[:5]}; "
          f"free-running stream first divergence {first} (oracle top-2 gap there {gap}); "
          f"{timing['output_tps']:.1f} tok/s", flush=True)
    if first is not None:
        # the free-running streams part only where the teacher-forced step
        # at that position was itself a near-tie
        assert any(i == first for i, _, _ in flips) or gap <= 0.5, (first, gap)
    assert np.mean(within) > 0.5


def test_cfg3_cfg_pair_1024_sampled(pair):
    engine, model, oracle = pair
    rng = np.random.default_rng(2003)
    cond = rng.integers(0, V, size=512).tolist()
    uncond = rng.integers(0, V, size=512).tolist()
    sampling = dict(temperature=1.0, top_p=0.93, top_k=50, repetition_penalty=1.0,
                    penalty_window=50, min_tokens=0, max_tokens=1024)
    seed, n, cfg = 77, 1024, 1.5
    cap = 512 + n + 8
    s = engine.session(2, cap)
    logits = np.stack([s.prefill(0, cond), s.prefill(1, uncond)])
    kv0 = [[s.read_kv(layer, b, 512) for layer in range(LAYERS)] for b in range(2)]
    o_sampling = oracle.sampling_struct(**sampling)
    tokens, g_step = [], {}
    stretch = 4  # steps compared with the oracle run from the prefill cache
    for step in range(n):
        tok = s.sample(sampling, seed, step, history=tokens, cfg_scale=cfg)
        x = oracle.guided_logits(logits[0], logits[1], cfg)
        scores = oracle.distribution(x, o_sampling, tokens, step)
        want = oracle.draw(scores, 1.0, seed, step)
        assert tok == want, (step, tok, want)
        tokens.append(tok)
        if step == n - 1:
            kv_end = [[s.read_kv(layer, b, 512 + step) for layer in range(LAYERS)]
                      for b in range(2)]
        logits = s.step([tok, tok])
        if step < stretch:
            g_step[step] = logits
    assert len(set(tokens)) > 50  # a sampled stream, not a repeated token
    print(f"[cfg3] {n} sampled tokens identical to the oracle's draws", flush=True)
    # a stretch after the prefill: the oracle decodes from the GPU's prefill
    # cache with the same tokens
    for b in range(2):
        ref = {}
        for mode in (0, 1):
            oracle.lib().oracle_set_accumulation(mode)
            try:
                cache = model.cache(cap)
                for layer, (k, v) in enumerate(kv0[b]):
                    cache.keys(layer)[:, :512] = k
                    cache.values(layer)[:, :512] = v
                cache.offset = 512
                ref[mode] = [model.step(t, cache) for t in tokens[:stretch]]
            finally:
                oracle.lib().oracle_set_accumulation(0)
        for i in range(stretch):
            check_fidelity(g_step[i][b], ref[0][i], ref[1][i])
    # the last step at KV 1536 from the GPU's cache
    for b in range(2):
        ref = oracle_step_from(model, oracle, kv_end[b], 512 + n - 1, tokens[-1], cap)
        check_fidelity(logits[b], ref[0], ref[1])
    s.close()


def test_cfg4_prefill_3000_decode_to_kv_8192(pair):
    engine, model, oracle = pair
    rng = np.random.default_rng(2004)
    prompt = rng.integers(0, V, size=3000).tolist()
    greedy = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                  penalty_window=50, min_tokens=0, max_tokens=5200)
    s = engine.session(1, 8200)
    s.prefill(0, prompt)
    steps = 8191 - 3000
    print(f"[cfg4] {steps} device-side greedy steps to KV 8191", flush=True)
    _, toks = s.time_generate(greedy, 0, steps, reset=True)
    assert s.position(0) == 8191
    kv = [s.read_kv(layer, 0, 8191) for layer in range(LAYERS)]
    token = int(rng.integers(0, V))
    gpu = s.step(token)[0]  # the step at KV 8192
    s.close()
    ref = oracle_step_from(model, oracle, kv, 8191, token, 8200)
    check_fidelity(gpu, ref[0], ref[1])


def test_cfg5_batch8_prompts_128_to_2048_capacity_6144(pair):
    engine, model, oracle = pair
    rng = np.random.default_rng(2005)
    B, cap = 8, 6144
    lens = rng.integers(128, 2049, size=B)
    s = engine.session(B, cap)
    for b, n in enumerate(lens):
        s.prefill(b, rng.integers(0, V, size=int(n)).tolist())
    greedy = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                  penalty_window=50, min_tokens=0, max_tokens=32)
    s.time_generate(greedy, 5, 16, reset=True)  # 16 batched device steps
    pos = [s.position(b) for b in range(B)]
    assert pos == [int(n) + 16 for n in lens]
    kv = [[s.read_kv(layer, b, pos[b]) for layer in range(LAYERS)] for b in range(B)]
    toks = rng.integers(0, V, size=B).tolist()
    gpu = s.step(toks)
    s.close()
    for b in range(B):
        print(f"[cfg5] sequence {b}: KV {pos[b] + 1}", flush=True)
        ref = oracle_step_from(model, oracle, kv[b], pos[b], toks[b], cap)
        check_fidelity(gpu[b], ref[0], ref[1])
