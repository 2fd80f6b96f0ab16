"""The oracle against the reference's own known answers (CPU).

Each case restates a reference test: tests/test_ar.py:10-19 (SwiGLU),
tests/test_sampling.py:37-122 (distribution filters, CFG arithmetic),
vendor/yue/tests/test_fast.py:136-149 + fast.py:196-204 (window penalty),
tests/test_cache.py:9-42 and vendor/yue/tests/test_model.py:54-139 (cache
semantics, chunked prefill, causality).
"""
import numpy as np
import pytest

from conftest import TINY

EOD, ABC_END, MUSIC_END, CODEC_OFFSET, CODEC_SIZE, VOCAB = (151643, 151848, 151852, 151853,
                                                            32768, 184704)


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


def test_swiglu_fp32_silu_before_bf16_product(oracle):
    # tests/test_ar.py:10-19 (weights = 1 makes the MLP bf16(silu(x)) * x)
    x = bf([-16, -5, -2.71875, -.1875, 0, .1875, 2.71875, 5, 16])
    expected = [2.8848648071289062e-05, 0.1669921875, 0.45703125, 0.015869140625, 0.0,
                0.019287109375, 6.9375, 24.875, 256.0]
    np.testing.assert_array_equal(oracle.bf16_to_f32(oracle.silu_mul(x, x)), expected)


@pytest.mark.parametrize("scale,expected", [
    (1.01, [4.5625, -3.3125, 0.004150390625, 18.5]),  # test_sampling.py:103-109
    (1.5, [7.375, -6.25, 0.013671875, 19.25]),
])
def test_cfg_uses_bf16_rounding_points(oracle, scale, expected):
    c = bf([4.5, -3.25, 0.00390625, 18.5])
    u = bf([-1.25, 2.75, -0.015625, 17.0])
    np.testing.assert_array_equal(oracle.bf16_to_f32(oracle.guided_logits(c, u, scale)), expected)


def semantic_logits(values, fill=-20.0):
    logits = np.full(CODEC_SIZE + 1, fill, dtype=np.float32)
    logits[1:1 + len(values)] = values  # native CODEC_OFFSET + i -> local 1 + i
    return bf(logits)


def test_topk_keeps_all_ties_at_the_cut(oracle):
    # test_sampling.py:37-41
    s = oracle.sampling_struct(top_k=2, top_p=1, min_tokens=0, repetition_penalty=1)
    scores = oracle.distribution(semantic_logits([5, 4, 4, 3]), s, [], 0, "semantic")
    assert np.flatnonzero(np.isfinite(scores)).tolist() == [1, 2, 3]


@pytest.mark.parametrize("legacy,kept", [(False, [1]), (True, [1, 2, 3])])
def test_shifted_nucleus_and_mode_specific_minimum(oracle, legacy, kept):
    # test_sampling.py:44-49
    s = oracle.sampling_struct(top_k=4, top_p=.01, min_tokens=0, repetition_penalty=1)
    scores = oracle.distribution(semantic_logits([5, 4, 3, 2]), s, [], 0, "semantic", legacy)
    assert np.flatnonzero(np.isfinite(scores)).tolist() == kept


def test_legacy_nucleus_equal_logits_keeps_three(oracle):
    # test_sampling.py:52-63
    s = oracle.sampling_struct(top_k=4, top_p=.749, min_tokens=0, repetition_penalty=1)
    scores = oracle.distribution(semantic_logits([0, 0, 0, 0], fill=-np.inf), s, [], 0,
                                 "semantic", True)
    assert int(np.isfinite(scores).sum()) == 3


def head_model(oracle, rows):
    """A hidden-size-1 model whose lm_head holds `rows` (test_sampling.py:85-99)."""
    cfg = dict(hidden_size=1, intermediate_size=1, num_hidden_layers=0, num_attention_heads=1,
               num_key_value_heads=1, head_dim=2, vocab_size=VOCAB, rms_norm_eps=1e-6,
               rope_theta=1e6, qk_norm=True)
    w = {"model.embed_tokens.weight": np.zeros((VOCAB, 1), np.uint16),
         "model.norm.weight": bf([1.0]), "lm_head.weight": bf(rows).reshape(VOCAB, 1)}
    return oracle.Model(cfg, w)


@pytest.mark.parametrize("phase,content,end", [
    ("abc", EOD - 1, ABC_END),
    ("semantic", CODEC_OFFSET + CODEC_SIZE - 1, MUSIC_END),
])
def test_projected_rows_and_min_tokens_under_greedy(oracle, phase, content, end):
    # test_sampling.py:85-110: the excluded EOD row and trailing rows never win
    rows = np.zeros(VOCAB, np.float32)
    rows[content], rows[end], rows[EOD], rows[-1] = 3, 4, 100, 101
    model = head_model(oracle, rows)
    logits = model.project(bf([2.0]), phase)
    assert logits.size == (EOD + 1 if phase == "abc" else CODEC_SIZE + 1)
    s = oracle.sampling_struct(temperature=0, top_k=1, top_p=.01, min_tokens=1)
    for step, expected in ((0, content), (1, end)):
        scores = oracle.distribution(logits, s, [], step, phase)
        local = oracle.draw(scores, 0.0, 0, step)
        assert oracle.lib().oracle_local_to_native(local, oracle.PHASES[phase]) == expected


def test_window_penalty_counts_expire_and_keep_sign(oracle):
    # test_sampling.py:94-100 / 113-119: window 3 of [C+2]*5 + [C, C, C+1]
    C = CODEC_OFFSET
    history = [C + 2] * 5 + [C, C, C + 1]
    s = oracle.sampling_struct(temperature=.7, top_p=1, top_k=20, min_tokens=0,
                               repetition_penalty=1.2, penalty_window=3)
    scores = oracle.distribution(semantic_logits([4.5, -4.5, 3]), s, history, 0, "semantic")
    p, t = np.float32(1.2), np.float32(.7)
    # local 1 seen twice (divided by 1.2^2), local 2 once (negative: multiplied),
    # local 3 outside the window; then temperature; the -20 plateau ties survive
    assert scores[1] == (np.float32(4.5) / (p * p)) / t
    assert scores[2] == (np.float32(-4.5) * p) / t
    assert scores[3] == np.float32(3) / t
    assert np.isfinite(scores).all()


@pytest.mark.parametrize("history,penalty,expected", [
    ([2, 2, 3], 2.0, [0, 9, 3, -4]),   # vendor test_fast.py:136-149
    ([1], 3.0, [0, 3, 12, -2]),
])
def test_window_penalty_lookup_answers(oracle, history, penalty, expected):
    s = oracle.sampling_struct(temperature=0, top_p=1, top_k=4, min_tokens=0,
                               repetition_penalty=penalty, penalty_window=3)
    scores = oracle.distribution(bf([0, 9, 12, -2]), s, history, 0, "full")
    np.testing.assert_array_equal(scores, expected)


def test_min_tokens_masks_only_before_the_budget(oracle):
    s = oracle.sampling_struct(temperature=0, top_k=1, top_p=1, min_tokens=2,
                               repetition_penalty=1)
    logits = semantic_logits([1.0])
    logits[0] = bf([50.0])[0]  # the end row (local 0) would win
    assert oracle.draw(oracle.distribution(logits, s, [], 1, "semantic"), 0, 0, 1) == 1
    assert oracle.draw(oracle.distribution(logits, s, [], 2, "semantic"), 0, 0, 2) == 0


# ---- cache semantics (test_cache.py, test_model.py) ----

@pytest.fixture(scope="module")
def tiny(oracle):
    import yuear
    return oracle.Model(TINY, yuear.random_weights(TINY, 5, 0.02, 0.1))


def test_append_then_overflow_does_not_mutate(tiny):
    cache = tiny.cache(5)
    tiny.hidden([1, 2, 3], cache)
    tiny.hidden([4, 5], cache)
    keys = tiny_keys = cache.keys(0).copy()
    with pytest.raises(ValueError):
        tiny.hidden([6], cache)
    assert cache.offset == 5
    np.testing.assert_array_equal(cache.keys(0), tiny_keys)
    assert keys.shape == (2, 5, 128)


def test_chunked_prefill_equals_full_prefill(tiny):
    # bottom-right causal alignment (test_cache.py:24-30, test_model.py:54-64)
    ids = [3, 5, 8, 7, 4, 9]
    full = tiny.hidden(ids, tiny.cache(8))
    cache = tiny.cache(8)
    parts = [tiny.hidden(ids[a:b], cache) for a, b in ((0, 2), (2, 5), (5, 6))]
    np.testing.assert_array_equal(np.concatenate(parts), full)


def test_reset_hides_stale_tail(tiny):
    cache = tiny.cache(8)
    tiny.hidden([9, 9, 9, 9, 9, 9, 9], cache)
    cache.offset = 0
    np.testing.assert_array_equal(tiny.hidden([3, 4], cache), tiny.hidden([3, 4], tiny.cache(8)))


def test_causality_future_tokens_do_not_leak(tiny):
    # test_model.py:132-139
    a = tiny.hidden([3, 5, 8, 7], tiny.cache(4))
    b = tiny.hidden([3, 5, 12, 19], tiny.cache(4))
    np.testing.assert_array_equal(a[:2], b[:2])


def test_invalid_ids_and_capacity_are_rejected(oracle, tiny):
    with pytest.raises(ValueError):
        tiny.hidden([TINY["vocab_size"]], tiny.cache(4))
    with pytest.raises(ValueError):
        tiny.cache(0)
    with pytest.raises(ValueError):
        tiny.cache(24577)
