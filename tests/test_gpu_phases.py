"""The phase-sliced lm_head at the YuE2 vocabulary on the GPU vs the oracle.

ARModel::project (ar.cpp:302-323) scores only the rows a phase can emit:
"abc" the rows [0, EOD) plus the ABC_END row (local id EOD), "semantic" the
MUSIC_END row (local 0) plus the codec rows [CODEC_OFFSET, CODEC_OFFSET +
CODEC_SIZE). Model: one layer of the 3B shape (hidden 3072, 24/8 heads, FFN
8192) with the YuE2 vocabulary (184704 rows), N(0, 0.02) weights. After a
prefill and after one decode step, every phase's logits are compared with
oracle.project(h, phase) under the logit tolerance (2e-2 abs +
1e-2 rel: one layer, where it holds), and the abc / semantic slices must be
bit-identical to the same rows of the GPU's own full projection.
"""
import numpy as np
import pytest

from conftest import MODEL_3B

pytestmark = pytest.mark.gpu

EOD, ABC_END, MUSIC_END, CODEC_OFFSET, CODEC_SIZE, VOCAB = (151643, 151848, 151852, 151853,
                                                            32768, 184704)
CFG = dict(MODEL_3B, num_hidden_layers=1, vocab_size=VOCAB)


def f32(oracle, bits):
    return oracle.bf16_to_f32(bits).astype(np.float64)


def rows_of(full, phase):
    if phase == "abc":
        return np.concatenate([full[:EOD], full[ABC_END:ABC_END + 1]])
    return np.concatenate([full[MUSIC_END:MUSIC_END + 1],
                           full[CODEC_OFFSET:CODEC_OFFSET + CODEC_SIZE]])


@pytest.fixture(scope="module")
def pair(yuear_lib, oracle):
    w = yuear_lib.random_weights(CFG, 184704)
    engine = yuear_lib.Engine(CFG, w)
    model = oracle.Model(CFG, w)
    yield engine, model
    engine.close()


def test_phase_slices_match_oracle_and_full_rows(pair, oracle):
    engine, model = pair
    rng = np.random.default_rng(11)
    prefix = [151851, 151853] + rng.integers(CODEC_OFFSET, VOCAB, size=9).tolist()
    token = int(rng.integers(CODEC_OFFSET, VOCAB))
    got = {}
    for phase in ("full", "abc", "semantic"):
        s = engine.session(1, 32, phase)
        size = {"full": VOCAB, "abc": EOD + 1, "semantic": CODEC_SIZE + 1}[phase]
        assert s.vocab == size == model.phase_size(phase)
        got[phase] = [s.prefill(0, prefix), s.step(token)[0]]
        s.close()
        cache = model.cache(32)
        ref = [model.prefill(prefix, cache, phase), model.step(token, cache, phase)]
        for g, r in zip(got[phase], ref):
            assert g.shape == r.shape == (size,)
            gf, rf = f32(oracle, g), f32(oracle, r)
            err = np.abs(gf - rf)
            print(f"[phases] {phase}: max |logit| {np.abs(rf).max():.3f}, max err {err.max():.4f}, "
                  f"argmax {gf.argmax()} / {rf.argmax()}", flush=True)
            assert (err <= 2e-2 + 1e-2 * np.abs(rf)).all()
    for phase in ("abc", "semantic"):
        for g, full in zip(got[phase], got["full"]):
            np.testing.assert_array_equal(g, rows_of(full, phase))


def test_generate_tokens_abc_phase_draws_match_oracle(pair, oracle):
    """generate_tokens in the abc phase (151644 rows: the sampler spread over
    workgroups, the end row in the partial last chunk) with the ABC sampling
    defaults, a penalty window and min_tokens: every token equals the
    oracle's distribution + draw on the GPU's own logits, replayed step by
    step through a session (the same kernels)."""
    engine, _ = pair
    rng = np.random.default_rng(5)
    prefix = [EOD] + rng.integers(0, EOD, size=12).tolist()
    sampling = dict(temperature=0.7, top_p=0.9, top_k=30, repetition_penalty=1.005,
                    penalty_window=100, min_tokens=6, max_tokens=24)
    seed = 77
    tokens, _, _ = engine.generate_tokens(prefix, sampling, seed, phase="abc")
    assert 6 <= len(tokens) <= 24
    assert ABC_END not in tokens[:6]
    s = engine.session(1, len(prefix) + 32, "abc")
    logits = s.prefill(0, prefix)
    ref = oracle.sampling_struct(**sampling)
    for step, token in enumerate(tokens):
        scores = oracle.distribution(logits, ref, tokens[:step], step, "abc")
        local = oracle.draw(scores, sampling["temperature"], seed, step)
        assert oracle.lib().oracle_local_to_native(local, oracle.PHASES["abc"]) == token, step
        if token == ABC_END:
            break
        logits = s.step(token)[0]
    s.close()
