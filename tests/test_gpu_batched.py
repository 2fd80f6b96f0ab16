"""Batched decode (3..8 independent sequences on the MFMA GEMV) on the GPU.

Each sequence of a batched step is compared with the oracle running that
sequence alone (native/src/ar.cpp:246-323 decode step; the sequences are
independent requests of sampling.cpp:185-288), and sequences must not
interact: branch b of a mixed batch equals branch b of a batch of copies.
"""
import numpy as np
import pytest

from conftest import MODEL_3B, check_fidelity

pytestmark = pytest.mark.gpu

TWO_LAYER = dict(MODEL_3B, num_hidden_layers=2)
HIDDEN_2048 = dict(hidden_size=2048, intermediate_size=6144, num_hidden_layers=3,
                   num_attention_heads=16, num_key_value_heads=8, head_dim=128, vocab_size=8192,
                   max_position_embeddings=4096, rms_norm_eps=1e-6, rope_theta=1e6, qk_norm=True)


@pytest.fixture(scope="module")
def engine(yuear_lib):
    e = yuear_lib.Engine(TWO_LAYER, None, seed=11)
    yield e
    e.close()


GREEDY = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0, penalty_window=50,
              min_tokens=0, max_tokens=64)
SAMPLED = dict(temperature=0.9, top_p=0.9, top_k=40, repetition_penalty=1.1, penalty_window=20,
               min_tokens=0, max_tokens=64)


@pytest.mark.parametrize("sampling", [GREEDY, SAMPLED], ids=["greedy", "sampled"])
def test_independent_branches_do_not_interact(engine, sampling):
    # More than two branches decode as independent sequences: branch b draws
    # its own token from its own logits, history and seed + b. Branch b of a
    # 3-branch session with mixed prompts must equal branch b of a 3-branch
    # session whose branches all hold prompt b (same kernels, same column of
    # every batched product), compared through the KV each step appends.
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, 83968, size=n).tolist() for n in (40, 17, 63)]
    steps, seed = 12, 99

    def decode(branch_prompts):
        s = engine.session(3, 128)
        for b, pr in enumerate(branch_prompts):
            s.prefill(b, pr)
        s.time_generate(sampling, seed, steps, reset=True)
        pos = [s.position(b) for b in range(3)]
        kv = [s.read_kv(1, b, pos[b]) for b in range(3)]
        s.close()
        return pos, kv

    pos, got = decode(prompts)
    assert pos == [len(pr) + steps for pr in prompts]
    for b, pr in enumerate(prompts):
        _, want = decode([pr] * 3)
        np.testing.assert_array_equal(got[b][0], want[b][0])
        np.testing.assert_array_equal(got[b][1], want[b][1])


@pytest.mark.parametrize("branches", [5])
def test_batched_steps_match_oracle(yuear_lib, oracle, branches):
    # Hidden-2048 model (K 2048 / 6144 on MFMA at 3..8 sequences): each
    # sequence's step logits against the oracle run alone, under the fidelity
    # rule for multi-layer models (fp32 vs fp64 accumulation radius).
    w = yuear_lib.random_weights(HIDDEN_2048, 8)
    engine = yuear_lib.Engine(HIDDEN_2048, w)
    model = oracle.Model(HIDDEN_2048, w)
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, 8192, size=n).tolist() for n in (33, 7, 120, 64, 2)][:branches]
    toks = rng.integers(0, 8192, size=(3, branches))
    s = engine.session(branches, 256)
    for b, pr in enumerate(prompts):
        s.prefill(b, pr)
    got = np.stack([s.step(t.tolist()) for t in toks])
    s.close()
    engine.close()
    try:
        for b, pr in enumerate(prompts):
            want = {}
            for mode in (0, 1):
                oracle.lib().oracle_set_accumulation(mode)
                cache = model.cache(256)
                model.prefill(pr, cache)
                want[mode] = [model.step(int(t[b]), cache) for t in toks]
            for i in range(len(toks)):
                print(f"branch {b} step {i}", flush=True)
                check_fidelity(got[i, b], want[0][i], want[1][i])
    finally:
        oracle.lib().oracle_set_accumulation(0)


@pytest.mark.parametrize("branches", [3, 8])
def test_batched_layer_matches_oracle_per_sequence(yuear_lib, oracle, branches):
    # Batches of 3..8 sequences run their projections on MFMA: each sequence
    # of one 3072-wide layer step (own KV of its own length, own input) must
    # match the oracle's single-sequence layer within the logits tolerance.
    from make_golden import LAYER
    seed = 3
    w = yuear_lib.random_weights(LAYER, seed)
    engine = yuear_lib.Engine(LAYER, w)
    model = oracle.Model(LAYER, w)
    lengths = [511, 64, 300, 1, 200, 129, 17, 450][:branches]
    x = yuear_lib.random_normal(seed, 901, (branches, 3072))
    s = engine.session(branches, 512)
    kvs = []
    for b, n in enumerate(lengths):
        kv = yuear_lib.random_normal(seed, 900 + 10 * b, (2, 8, n - 1, 128)) if n > 1 else None
        if kv is not None:
            s.write_kv(0, b, kv[0], kv[1])
        kvs.append(kv)
    got = s.layer_step(0, x)
    for b, n in enumerate(lengths):
        cache = model.cache(512)
        if kvs[b] is not None:
            cache.keys(0)[:, :n - 1] = kvs[b][0]
            cache.values(0)[:, :n - 1] = kvs[b][1]
        cache.offset = n - 1
        want = model.layer(0, x[b:b + 1], cache)[0]
        g, r = oracle.bf16_to_f32(got[b]), oracle.bf16_to_f32(want)
        assert (np.abs(g - r) <= 2e-2 + 1e-2 * np.abs(r)).all(), f"branch {b}"
        assert np.mean(got[b] == want) > 0.6, f"branch {b}"
        assert s.position(b) == n
    s.close()
    engine.close()


def test_sample_rejects_batched_sessions(engine):
    s = engine.session(3, 16)
    with pytest.raises(ValueError, match="independently"):
        s.sample(GREEDY, 1, 0)
    s.close()
