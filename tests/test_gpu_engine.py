"""Engine / session / generate_tokens on the GPU vs the oracle and the golden
vectors (tiny model of the 3B layer family, one 3B-shaped layer).

Reference behaviour restated: vendor/yue/tests/test_cuda_graph.py:38-115
(decode-step equations, cache poisoning, branch isolation, lifecycle,
capacity validation), tests/test_cache.py (append/overflow), and the
fidelity methodology of tools/fidelity.py:124-148 (max_abs, argmax).
"""
import os

import numpy as np
import pytest

from conftest import ROOT, TINY

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(ROOT, "tests", "golden")
ATOL, RTOL = 2e-2, 1e-2  # logits tolerance of the decode path (bf16, fp32 accumulate)


def f(b):
    import cpu_ref
    return cpu_ref.bf16_to_f32(b)


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


def within(a, b, atol=ATOL, rtol=RTOL):
    return np.abs(f(a) - f(b)) <= atol + rtol * np.abs(f(b))


@pytest.fixture(scope="module")
def tiny(yuear_lib, oracle):
    g = np.load(os.path.join(GOLDEN, "tiny_model.npz"))
    w = yuear_lib.random_weights(TINY, int(g["seed"]), float(g["std"]), float(g["norm_std"]))
    return yuear_lib.Engine(TINY, w), oracle.Model(TINY, w), g


def test_tiny_prefill_and_steps_match_oracle_and_golden(tiny):
    engine, model, g = tiny
    s = engine.session(1, 16)
    cache = model.cache(16)
    got = [s.prefill(0, g["prefix"].tolist())]
    want = [model.prefill(g["prefix"].tolist(), cache)]
    for t in g["steps"]:
        got.append(s.step(int(t))[0])
        want.append(model.step(int(t), cache))
    got, want = np.stack(got), np.stack(want)
    assert within(got, want).all()
    assert within(got, g["logits_bf16"]).all()
    assert (f(got).argmax(1) == f(g["logits_bf16"]).argmax(1)).all()
    # The attention sums 32 keys per MFMA where the oracle sums key by key:
    # ~0.05 % of attention outputs round to the neighbouring bf16, and two
    # layers spread such changes over many logits as a few units of their
    # last place. Every logit stays within one bf16 unit of the logits' scale
    # (2^-8 of max |logit|) of the oracle's.
    err = np.abs(f(got) - f(want))
    assert (err <= 2.0 ** -8 * np.abs(f(want)).max()).all()
    assert s.position(0) == len(g["prefix"]) + len(g["steps"])


def test_model_without_qk_norm_matches_oracle(yuear_lib, oracle):
    # q/k RMSNorm off (no gains): the prefill's q/k preparation and the decode
    # attention's prologue apply RoPE only
    cfg = dict(TINY, qk_norm=False)
    w = yuear_lib.random_weights(cfg, 5, 0.02, 0.1)
    engine, model = yuear_lib.Engine(cfg, w), oracle.Model(cfg, w)
    rng = np.random.default_rng(5)
    prefix = rng.integers(0, cfg["vocab_size"], 37).tolist()
    s = engine.session(1, 48)
    cache = model.cache(48)
    got, want = [s.prefill(0, prefix)], [model.prefill(prefix, cache)]
    for t in rng.integers(0, cfg["vocab_size"], 5):
        got.append(s.step(int(t))[0])
        want.append(model.step(int(t), cache))
    s.close()
    engine.close()
    assert within(np.stack(got), np.stack(want)).all()


# (hidden, intermediate, layers, heads, kv heads, vocab, qk_norm, branches):
# widths that are and are not the batched MFMA form's (2048 / 3072 / 6144 /
# 8192), every accepted heads-per-kv-head ratio, one to five branches
RANDOM_MODELS = [
    (64, 128, 1, 1, 1, 300, True, 1),
    (320, 704, 2, 6, 1, 1000, False, 2),
    (1024, 1536, 3, 8, 2, 4099, True, 3),
    (2048, 6144, 1, 16, 8, 2048, True, 5),
    (576, 2048, 2, 24, 8, 777, False, 4),
    (1536, 512, 1, 32, 4, 3000, True, 2),
]


@pytest.mark.parametrize("model", RANDOM_MODELS, ids=[f"h{m[0]}-f{m[1]}-l{m[2]}-{m[3]}x{m[4]}-b{m[7]}"
                                                      for m in RANDOM_MODELS])
def test_random_model_shapes_match_oracle(yuear_lib, oracle, model):
    # the engine across model shapes (ar.cpp:133-245 configs): per-branch
    # prefills of random lengths, then batched steps. Every prefill, and
    # every step recomputed by the oracle from the GPU's own cache, within
    # the per-logit bound; the oracle decoding from its own cache drifts by
    # the caches' bf16 rounding differences (a few units of the logits' last
    # place on a handful of logits), so against it nearly every logit is
    # within the bound and none further than 4 bf16 units of the scale
    H, F, layers, hq, hkv, vocab, qk_norm, branches = model
    cfg = dict(hidden_size=H, intermediate_size=F, num_hidden_layers=layers,
               num_attention_heads=hq, num_key_value_heads=hkv, head_dim=128, vocab_size=vocab,
               max_position_embeddings=512, rms_norm_eps=1e-5, rope_theta=5e5, qk_norm=qk_norm)
    rng = np.random.default_rng(H + F + hq)
    w = yuear_lib.random_weights(cfg, int(rng.integers(0, 1000)), 0.02, 0.1)
    engine, ref = yuear_lib.Engine(cfg, w), oracle.Model(cfg, w)
    cap = 320
    s = engine.session(branches, cap)
    caches = [ref.cache(cap) for _ in range(branches)]
    lens = []
    for b in range(branches):
        prefix = rng.integers(0, vocab, int(rng.integers(1, 300))).tolist()
        lens.append(len(prefix))
        got, want = s.prefill(b, prefix), ref.prefill(prefix, caches[b])
        assert within(got, want).all(), ("prefill", b)
    for step in range(4):
        toks = [int(t) for t in rng.integers(0, vocab, branches)]
        kv = [[s.read_kv(layer, b, lens[b] + step) for layer in range(layers)]
              for b in range(branches)]
        got = s.step(toks)
        for b in range(branches):
            mine = ref.cache(cap)
            for layer, (k, v) in enumerate(kv[b]):
                mine.keys(layer)[:, :lens[b] + step] = k
                mine.values(layer)[:, :lens[b] + step] = v
            mine.offset = lens[b] + step
            assert within(got[b], ref.step(toks[b], mine)).all(), ("step from GPU cache", step, b)
            want = ref.step(toks[b], caches[b])
            err = np.abs(f(got[b]) - f(want))
            assert np.mean(within(got[b], want)) >= 0.99, ("step", step, b)
            assert err.max() <= 2.0 ** -6 * np.abs(f(want)).max(), ("step", step, b, err.max())
    s.close()
    engine.close()


def test_repeated_runs_are_bit_identical(yuear_lib):
    # every reduction has a fixed order (the attention's split merge adds the
    # splits in split order whichever workgroup arrives last, the GEMV
    # butterflies and the GEMM's K loop are fixed): two sessions fed the same
    # prompts and tokens give the same bits, prefill and every decode step,
    # at one branch, the CFG pair and five branches (the MFMA form), with the
    # 3B layer shape and ~17 attention splits per kv head
    cfg = dict(hidden_size=3072, intermediate_size=8192, num_hidden_layers=2,
               num_attention_heads=24, num_key_value_heads=8, head_dim=128, vocab_size=4096,
               max_position_embeddings=4096, rms_norm_eps=1e-5, rope_theta=5e5, qk_norm=True)
    engine = yuear_lib.Engine(cfg, seed=7)
    rng = np.random.default_rng(7)
    for branches in (1, 2, 5):
        prompts = [rng.integers(0, 4096, int(rng.integers(500, 2000))).tolist()
                   for _ in range(branches)]
        toks = rng.integers(0, 4096, size=(12, branches))
        runs = []
        for _ in range(2):
            s = engine.session(branches, 2100)
            out = [s.prefill(b, p) for b, p in enumerate(prompts)]
            out += [s.step([int(t) for t in row]) for row in toks]
            runs.append(out)
            s.close()
        for i, (a, b) in enumerate(zip(*runs)):
            np.testing.assert_array_equal(a, b, err_msg=f"branches {branches}, output {i}")
    engine.close()


def test_prefill_fused_reduce_norm_is_bit_identical(yuear_lib, monkeypatch):
    # A split residual GEMM (o_proj, down) and the RMSNorm after it run as one
    # kernel (gemm_reduce_norm_kernel); YUEAR_PREFILL_FUSE_NORM=0 keeps the
    # reduce kernel and the row norm apart. At the 3B layer shape both
    # projections split at 100 and 700 tokens and down alone at 1024: prefill
    # logits and the decode steps after it must be the same bits either way.
    cfg = dict(hidden_size=3072, intermediate_size=8192, num_hidden_layers=2,
               num_attention_heads=24, num_key_value_heads=8, head_dim=128, vocab_size=4096,
               max_position_embeddings=4096, rms_norm_eps=1e-5, rope_theta=5e5, qk_norm=True)
    engine = yuear_lib.Engine(cfg, seed=11)
    rng = np.random.default_rng(11)
    for n in (100, 700, 1024):
        prompt = rng.integers(0, 4096, n).tolist()
        toks = rng.integers(0, 4096, size=3)
        runs = []
        for fused in ("1", "0"):
            monkeypatch.setenv("YUEAR_PREFILL_FUSE_NORM", fused)
            s = engine.session(1, n + 8)
            runs.append([s.prefill(0, prompt)] + [s.step(int(t))[0] for t in toks])
            s.close()
        for i, (a, b) in enumerate(zip(*runs)):
            np.testing.assert_array_equal(a, b, err_msg=f"{n} tokens, output {i}")
    engine.close()


def test_chunked_prefill_is_bit_identical_to_one_pass(tiny):
    engine, _, _ = tiny
    ids = [5, 9, 14, 200, 33, 1, 511, 256, 3]
    a = engine.session(1, 32)
    full = a.prefill(0, ids)
    b = engine.session(1, 32)
    b.prefill(0, ids[:4])
    part = b.prefill(0, ids[4:])
    np.testing.assert_array_equal(full, part)
    for layer in range(TINY["num_hidden_layers"]):
        ka, va = a.read_kv(layer, 0, len(ids))
        kb, vb = b.read_kv(layer, 0, len(ids))
        np.testing.assert_array_equal(ka, kb)
        np.testing.assert_array_equal(va, vb)


def test_decode_step_agrees_with_prefill_path(tiny):
    engine, _, _ = tiny
    ids = [7, 8, 9, 10, 11, 12]
    a = engine.session(1, 16)
    via_prefill = a.prefill(0, ids)
    b = engine.session(1, 16)
    b.prefill(0, ids[:-1])
    via_step = b.step(ids[-1])[0]
    assert within(via_step, via_prefill).all()


def test_cache_poisoning_and_branch_isolation(tiny):
    # test_cuda_graph.py:62-79
    engine, _, _ = tiny
    prefixes = [[2, 3, 4, 5], [6]]
    sessions = []
    for _ in range(2):
        s = engine.session(2, 12)
        for b, p in enumerate(prefixes):
            s.prefill(b, p)
        sessions.append(s)
    base, changed = sessions
    for layer in range(TINY["num_hidden_layers"]):
        for b, p in enumerate(prefixes):
            k, v = changed.read_kv(layer, b, 12)
            k[:, len(p):] = bf(1000.0)
            v[:, len(p):] = bf(-1000.0)
            changed.write_kv(layer, b, k, v)
            changed.set_position(b, len(p))
    np.testing.assert_array_equal(changed.step(7), base.step(7))
    for layer in range(TINY["num_hidden_layers"]):  # perturb branch 0's visible cache
        k, v = changed.read_kv(layer, 0, 5)
        v[:, :2] = bf(f(v[:, :2]) + 1)
        changed.write_kv(layer, 0, k, v)
    old, new = base.step(8), changed.step(8)
    np.testing.assert_array_equal(new[1], old[1])
    assert not np.array_equal(new[0], old[0])


def test_lifecycle_and_capacity_errors(tiny):
    engine, _, _ = tiny
    s = engine.session(1, 5)
    s.prefill(0, [1, 2, 3])
    with pytest.raises(ValueError, match="capacity"):
        s.prefill(0, [4, 5, 6])
    assert s.position(0) == 3
    s.step(4)
    s.step(5)
    with pytest.raises(ValueError, match="budget"):
        s.step(6)
    with pytest.raises(ValueError):
        s.step(TINY["vocab_size"])
    with pytest.raises(ValueError):
        engine.session(1, 0)
    with pytest.raises(ValueError):
        engine.session(9, 8)
    s.close()
    with pytest.raises(RuntimeError, match="closed"):
        s.step(1)


def test_full_context_last_step_matches_oracle(yuear_lib, oracle):
    # a session of the whole 24576-token context (the capacity range of
    # ar.cpp:98-132): prefill to 24570, graph steps to the last slot 24575,
    # that step against the oracle decoding from the GPU's cache (RoPE's last
    # table row, every cache block), then the budget error with nothing moved
    cfg = dict(TINY, max_position_embeddings=24576)
    w = yuear_lib.random_weights(cfg, 11, 0.02, 0.1)
    engine, model = yuear_lib.Engine(cfg, w), oracle.Model(cfg, w)
    rng = np.random.default_rng(24576)
    n0, last = 24570, 24575
    s = engine.session(1, 24576)
    s.prefill(0, rng.integers(0, cfg["vocab_size"], n0).tolist())
    toks = [int(t) for t in rng.integers(0, cfg["vocab_size"], last - n0 + 1)]
    for t in toks[:-1]:
        s.step(t)
    assert s.position(0) == last
    kv = [s.read_kv(layer, 0, last) for layer in range(cfg["num_hidden_layers"])]
    got = s.step(toks[-1])[0]
    cache = model.cache(24576)
    for layer, (k, v) in enumerate(kv):
        cache.keys(layer)[:, :last] = k
        cache.values(layer)[:, :last] = v
    cache.offset = last
    want = model.step(toks[-1], cache)
    assert within(got, want).all()
    assert s.position(0) == 24576
    with pytest.raises(ValueError, match="budget"):
        s.step(1)
    assert s.position(0) == 24576
    s.close()
    engine.close()


def test_generate_tokens_greedy_matches_oracle_teacher_forced(tiny, oracle):
    engine, model, _ = tiny
    prefix = [3, 17, 255, 1, 98]
    sampling = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                    penalty_window=50, min_tokens=0, max_tokens=24)
    seen = []
    tokens, timing, truncated = engine.generate_tokens(
        prefix, sampling, 7, on_token=lambda phase, t: seen.append((phase, t)))
    assert len(tokens) == 24 and truncated and seen == [("full", t) for t in tokens]
    assert timing["output_tokens"] == 24 and timing["cfg_branches"] == 1
    assert set(timing) >= {"seconds", "prefill_seconds", "ttft_seconds", "output_tps",
                           "prefix_tokens", "execution", "attention", "backend"}
    cache = model.cache(len(prefix) + 24)
    logits = model.prefill(prefix, cache)
    s = oracle.sampling_struct(**sampling)
    for step, token in enumerate(tokens):
        scores = oracle.distribution(logits, s, tokens[:step], step, "full")
        want = oracle.draw(scores, 0.0, 7, step)
        if want != token:  # only a near-tie may differ (gap-aware accounting)
            top = np.sort(scores)[-2:]
            assert top[1] - top[0] <= 2 * (ATOL + RTOL * abs(top[1])), (step, token, want)
        logits = model.step(token, cache)


def test_generate_tokens_cfg_sampled_matches_oracle(tiny, oracle):
    engine, model, _ = tiny
    prefix, negative = [3, 17, 255, 1, 98, 400], [9, 8, 7]
    sampling = dict(temperature=1.0, top_p=0.93, top_k=50, repetition_penalty=1.0,
                    penalty_window=50, min_tokens=0, max_tokens=20)
    tokens, timing, _ = engine.generate_tokens(prefix, sampling, 1234, negative=negative,
                                               cfg_scale=1.5)
    assert timing["cfg_branches"] == 2 and len(tokens) == 20
    cp, cn = model.cache(40), model.cache(40)
    lp, ln = model.prefill(prefix, cp), model.prefill(negative, cn)
    s = oracle.sampling_struct(**sampling)
    agree = 0
    for step, token in enumerate(tokens):
        scores = oracle.distribution(oracle.guided_logits(lp, ln, 1.5), s, tokens[:step], step,
                                     "full")
        agree += oracle.draw(scores, 1.0, 1234, step) == token
        lp, ln = model.step(token, cp), model.step(token, cn)
    assert agree >= len(tokens) - 1


def test_generate_tokens_validation(tiny):
    engine, _, _ = tiny
    ok = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0, penalty_window=50,
              min_tokens=0, max_tokens=4)
    with pytest.raises(ValueError, match="negative"):
        engine.generate_tokens([1, 2], ok, 1, cfg_scale=1.5)
    with pytest.raises(ValueError, match="24576"):
        engine.generate_tokens([1] * 10, dict(ok, max_tokens=24570), 1)
    with pytest.raises(ValueError):
        engine.generate_tokens([], ok, 1)
    with pytest.raises(ValueError):
        engine.generate_tokens([1], dict(ok, top_p=0.0), 1)
    with pytest.raises(ValueError, match="seed"):
        engine.generate_tokens([1], ok, 2**63)
    with pytest.raises(ValueError, match="phase"):
        engine.generate_tokens([1], ok, 1, phase="lyrics")


def test_throwing_callback_cancels(tiny):
    engine, _, _ = tiny
    sampling = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                    penalty_window=50, min_tokens=0, max_tokens=30)
    calls = []

    def boom(phase, token):
        calls.append(token)
        if len(calls) == 3:
            raise KeyError("stop")

    with pytest.raises(KeyError):
        engine.generate_tokens([1, 2, 3], sampling, 3, on_token=boom)
    assert len(calls) == 3
    tokens, _, _ = engine.generate_tokens([1, 2, 3], sampling, 3)  # engine still usable
    assert len(tokens) == 30


def test_cancel_points_and_messages(yuear_lib):
    # the reference polls its Cancelled predicate after validation and at
    # the start of each prefill ("Cancelled before prefill", sampling.cpp:156,
    # 206), before every 1024-token prefill chunk ("Cancelled during prefill",
    # :164) and before every step ("Cancelled during <phase>", :243); the
    # library polls at the same points (its chunks hold up to 4096 tokens, so
    # a 9000-token prefix is three chunks) and reports nothing after a cancel
    cfg = dict(TINY, max_position_embeddings=16384)
    engine = yuear_lib.Engine(cfg, seed=3)
    prefix = [int(t) for t in np.random.default_rng(0).integers(0, cfg["vocab_size"], 9000)]
    sampling = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                    penalty_window=50, min_tokens=0, max_tokens=16)
    for answer_false, message in [(0, "Cancelled before prefill"),
                                  (1, "Cancelled before prefill"),
                                  (2, "Cancelled during prefill"),
                                  (4, "Cancelled during prefill"),
                                  (5, "Cancelled during full"),
                                  (8, "Cancelled during full")]:
        polls, calls, at_cancel = [], [], []

        def cancelled():
            polls.append(1)
            if len(polls) > answer_false and not at_cancel:
                at_cancel.append(len(calls))
            return len(polls) > answer_false

        with pytest.raises(InterruptedError, match=message):
            engine.generate_tokens(prefix, sampling, 1, cancelled=cancelled,
                                   on_token=lambda ph, tok: calls.append(tok))
        assert len(polls) == answer_false + 1  # no poll after the cancel
        assert len(calls) == at_cancel[0], (answer_false, calls)  # no token after it
        if answer_false < 5:
            assert not calls
    never = []
    tokens, _, _ = engine.generate_tokens(prefix, sampling, 1,
                                          cancelled=lambda: never.append(1) and False)
    assert len(tokens) == 16 and len(never) >= 5 + 16
    engine.close()


def test_end_token_and_min_tokens_in_semantic_phase(yuear_lib):
    # Zero layers' weights make the final hidden state the normalised
    # embedding (all ones), so logits are the row sums of lm_head: only the
    # end row (MUSIC_END) is positive. Greedy decoding must emit content until
    # min_tokens and then stop on the end token (sampling.cpp:47-50, 256-259).
    cfg = dict(hidden_size=64, intermediate_size=64, num_hidden_layers=1,
               num_attention_heads=1, num_key_value_heads=1, head_dim=128,
               vocab_size=184704, max_position_embeddings=256, rms_norm_eps=1e-5,
               rope_theta=1e6)
    w = {k: np.zeros(s, np.uint16) for k, s in yuear_lib.tensor_shapes(cfg).items()}
    w["model.embed_tokens.weight"][:] = 0x3F80
    for k in w:
        if k.endswith("norm.weight") or "layernorm" in k:
            w[k][:] = 0x3F80
    w["lm_head.weight"][151852] = bf(0.01)
    engine = yuear_lib.Engine(cfg, w)
    sampling = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.2,
                    penalty_window=50, min_tokens=5, max_tokens=40)
    tokens, timing, truncated = engine.generate_tokens([151851, 151853], sampling, 1,
                                                       phase="semantic")
    assert tokens == [151853] * 5 and not truncated
    assert timing["output_tokens"] == 6 and timing["content_tokens"] == 5


def test_3b_layer_step_matches_oracle_and_golden(yuear_lib, oracle):
    # one 3072-wide layer, KV N(0,1) over 511 slots, input N(0,1)
    from make_golden import LAYER
    g = np.load(os.path.join(GOLDEN, "layer_3072.npz"))
    seed, length = int(g["seed"]), int(g["length"])
    w = yuear_lib.random_weights(LAYER, seed)
    kv = yuear_lib.random_normal(seed, int(g["kv_stream"]), (2, 8, length - 1, 128))
    x = yuear_lib.random_normal(seed, int(g["x_stream"]), (1, 3072))
    engine = yuear_lib.Engine(LAYER, w)
    s = engine.session(1, length)
    s.write_kv(0, 0, kv[0], kv[1])
    got = s.layer_step(0, x)[0]
    model = oracle.Model(LAYER, w)
    cache = model.cache(length)
    cache.keys(0)[:, :length - 1] = kv[0]
    cache.values(0)[:, :length - 1] = kv[1]
    cache.offset = length - 1
    want = model.layer(0, x, cache)[0]
    assert within(got, want).all()
    assert within(got, g["hidden_bf16"]).all()
    assert np.mean(got == want) > 0.6
    assert s.position(0) == length
