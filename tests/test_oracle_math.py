"""The oracle against what the mathematics fixes (CPU).

Published known-answer vectors (Philox), closed forms and special cases
(bf16 rounding, RMSNorm, RoPE), fp64 brute force (linear, attention), and
the golden vectors of the upstream torch model for the composition of a
whole layer / model (tests/golden/make_golden.py). Each check is chosen so
that a plausible slip (dropped term, wrong sign or index, transposed
operand) fails it.
"""
import json
import os

import numpy as np
import pytest

from conftest import TINY

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")


def f(bits):
    import cpu_ref
    return cpu_ref.bf16_to_f32(bits)


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


# ---- Philox4x32-10 ----
# Random123 kat_vectors (Salmon et al., SC'11), philox4x32 10 rounds.
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize("ctr,key,out", KAT)
def test_philox_published_vectors(oracle, ctr, key, out):
    assert tuple(oracle.philox(ctr, key)) == out


def test_philox_matches_rocrand_fixture(oracle):
    path = os.path.join(GOLDEN, "philox_rocrand.json")
    vectors = json.load(open(path))
    assert len(vectors) >= 8
    for v in vectors:
        assert oracle.philox(v["ctr"], v["key"]) == v["out"]


# ---- bf16 rounding ----

def test_bf16_round_to_nearest_even():
    u = np.array([0x3F800000, 0x3F808000, 0x3F818000, 0x3F80C000, 0x3F807FFF, 0x7F800000,
                  0xFF800000, 0x80000000, 0x7F7FFFFF], dtype=np.uint32)
    got = bf(u.view(np.float32))
    # 1.0; tie -> even (down); tie -> even (up); above half; below half; inf;
    # -inf; -0; FLT_MAX overflows to inf under RNE
    assert got.tolist() == [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0x3F80, 0x7F80, 0xFF80, 0x8000,
                            0x7F80]
    nan = bf(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


# ---- portable log / exp used by the shared-draw protocol ----

def test_portable_log_and_exp_accuracy(oracle):
    lib = oracle.lib()
    xs = np.concatenate([np.geomspace(1e-30, 1e30, 4001), np.linspace(0.5, 2.0, 4001)])
    got = np.array([lib.oracle_plog(float(x)) for x in xs.astype(np.float32)], np.float64)
    ref = np.log(xs.astype(np.float32).astype(np.float64))
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1.0)) < 4e-7
    assert lib.oracle_plog(1.0) == 0.0
    ys = np.linspace(-87, 0, 8001).astype(np.float32)
    got = np.array([lib.oracle_pexp(float(y)) for y in ys], np.float64)
    ref = np.exp(ys.astype(np.float64))
    assert np.max(np.abs(got - ref) / ref) < 4e-7
    assert lib.oracle_pexp(0.0) == 1.0 and lib.oracle_pexp(-np.inf) == 0.0


def test_shared_uniform_is_in_open_unit_interval_and_flat(oracle):
    lib = oracle.lib()
    u = np.array([lib.oracle_uniform(17, s, i) for s in range(4) for i in range(2500)])
    assert u.min() > 0 and u.max() < 1
    assert abs(u.mean() - 0.5) < 0.01 and abs(np.mean(u < 0.25) - 0.25) < 0.01
    assert lib.oracle_uniform(17, 0, 0) != lib.oracle_uniform(2**40 + 17, 0, 0)


# ---- categorical draw ----
# sampling.cpp:128-132 draws categorical(log(softmax(scores))): token i with
# probability softmax(scores)_i. The oracle's draw (shared uniforms, argmax of
# s_i - log(-log u_i)) must produce exactly those frequencies after
# distribution() has applied the temperature (sampling.cpp:76-80).

def _chi2_pvalue(counts, probs):
    from scipy.stats import chisquare
    counts = np.asarray(counts, dtype=np.float64)
    return chisquare(counts, counts.sum() * np.asarray(probs, dtype=np.float64)).pvalue


def _draw_counts(oracle, scores, n_draws, key_of=None):
    """Token counts over (seed, step) pairs; key_of(scores, u) replaces the
    oracle's draw by a variant computed from the same uniforms."""
    lib = oracle.lib()
    counts = np.zeros(scores.size, dtype=np.int64)
    finite = np.isfinite(scores)
    for j in range(n_draws):
        seed, step = 9000 + j // 250, j % 250
        if key_of is None:
            tok = oracle.draw(scores, 1.0, seed, step)
        else:
            u = np.array([lib.oracle_uniform(seed, step, i) for i in range(scores.size)],
                         dtype=np.float64)
            key = np.where(finite, key_of(scores.astype(np.float64), u), -np.inf)
            tok = int(np.argmax(key))
        counts[tok] += 1
    return counts


@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_categorical_draw_follows_softmax(oracle, temperature):
    logits = bf([1.5, 0.25, -0.75, 2.0, 0.0, -30.0])
    sampling = oracle.sampling_struct(temperature=temperature, top_p=1.0, top_k=6,
                                      repetition_penalty=1.0, penalty_window=0, min_tokens=0)
    scores = oracle.distribution(logits, sampling, [], 0)
    lf = f(logits).astype(np.float64)
    assert np.allclose(scores, lf / temperature, rtol=1e-6)  # temperature applied once
    p = np.exp(lf / temperature - (lf / temperature).max())
    p /= p.sum()
    n = 40000
    counts = _draw_counts(oracle, scores, n)
    assert _chi2_pvalue(counts[:5], p[:5] / p[:5].sum()) > 1e-3, (counts, p * n)
    # slips the test must catch, drawn from the same uniforms: a sign-flipped
    # Gumbel term, and the temperature applied a second time
    flipped = _draw_counts(oracle, scores, 8000, lambda s, u: s + np.log(-np.log(u)))
    assert _chi2_pvalue(flipped[:5], p[:5] / p[:5].sum()) < 1e-6
    if temperature != 1.0:
        twice = _draw_counts(oracle, scores, 8000,
                             lambda s, u: s / temperature - np.log(-np.log(u)))
        assert _chi2_pvalue(twice[:5], p[:5] / p[:5].sum()) < 1e-6


def test_categorical_draw_skips_masked_rows_and_greedy_takes_lowest_index(oracle):
    scores = np.array([-np.inf, 0.5, -np.inf, 0.5, -np.inf], dtype=np.float32)
    seen = {oracle.draw(scores, 1.0, 5, s) for s in range(400)}
    assert seen == {1, 3}
    assert oracle.draw(scores, 0.0, 5, 0) == 1  # argmax ties: lowest index


# ---- model ops ----

def test_rms_norm_special_cases(oracle):
    w = bf(np.linspace(-2, 2, 64))
    # constant row 2 with eps -> 0: scale is exactly 1/2, y == w
    y = oracle.rms_norm(bf(np.full((1, 64), 2.0)), w, 1e-12)
    np.testing.assert_array_equal(y[0], w)
    y = oracle.rms_norm(bf(np.full((1, 64), -2.0)), w, 1e-12)
    np.testing.assert_array_equal(f(y[0]), -f(w))
    np.testing.assert_array_equal(f(oracle.rms_norm(np.zeros((1, 64), np.uint16), w, 1e-6)), 0)


def test_rms_norm_matches_fp64(oracle):
    rng = np.random.default_rng(3)
    x = bf(rng.normal(size=(16, 3072)) * 3)
    w = bf(1 + rng.normal(size=3072) * 0.1)
    xs = f(x).astype(np.float64)
    ref = xs / np.sqrt(np.mean(xs ** 2, axis=-1, keepdims=True) + 1e-5) * f(w)
    np.testing.assert_allclose(f(oracle.rms_norm(x, w, 1e-5)), ref, rtol=1.6e-2, atol=1e-6)


def test_linear_matches_fp64_and_one_hot(oracle):
    rng = np.random.default_rng(4)
    x = bf(rng.normal(size=(5, 3072)))
    w = bf(rng.normal(size=(257, 3072)) * 0.02)
    ref = f(x).astype(np.float64) @ f(w).astype(np.float64).T
    got = f(oracle.linear(x, w))
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-3)) < 8e-3
    eye = np.zeros((3072, 3072), np.uint16)
    eye[np.arange(3072), np.arange(3072)] = 0x3F80
    np.testing.assert_array_equal(oracle.linear(x, eye), x)
    perm = np.roll(np.arange(3072), 7)
    shuffled = np.zeros_like(eye)
    shuffled[np.arange(3072), perm] = 0x3F80
    np.testing.assert_array_equal(oracle.linear(x, shuffled), x[:, perm])


def test_rope_identity_at_zero_and_rotation(oracle):
    rng = np.random.default_rng(5)
    x = bf(rng.normal(size=(3, 4, 128)))
    np.testing.assert_array_equal(oracle.rope(x[:1], 0, 5e5), x[:1])
    out = f(oracle.rope(x, 100, 5e5)).astype(np.float64)
    xs = f(x).astype(np.float64)
    # fp64 half-split rotation at positions 100..102
    inv = 1.0 / (5e5 ** (np.arange(0, 128, 2) / 128))
    ang = (100 + np.arange(3))[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    ref = np.concatenate([xs[..., :64] * c - xs[..., 64:] * s,
                          xs[..., 64:] * c + xs[..., :64] * s], axis=-1)
    np.testing.assert_allclose(out, ref, atol=0.04, rtol=0.02)
    np.testing.assert_allclose(np.linalg.norm(out, axis=-1), np.linalg.norm(xs, axis=-1),
                               rtol=0.01)
    # swapping the halves (a classic slip) must not match
    wrong = np.concatenate([xs[..., :64] * c + xs[..., 64:] * s,
                            xs[..., 64:] * c - xs[..., :64] * s], axis=-1)
    assert np.max(np.abs(out - wrong)) > 0.5


def brute_attention(q, keys, values, offset):
    """fp64 softmax attention, GQA head h -> h // (Hq // Hkv)."""
    T, Hq, D = q.shape
    Hkv = keys.shape[0]
    out = np.zeros((T, Hq, D))
    for t in range(T):
        L = offset + t + 1
        for h in range(Hq):
            k = keys[h // (Hq // Hkv), :L].astype(np.float64)
            v = values[h // (Hq // Hkv), :L].astype(np.float64)
            s = (k @ q[t, h].astype(np.float64)) / np.sqrt(D)
            p = np.exp(s - s.max())
            out[t, h] = p @ v / p.sum()
    return out.reshape(T, Hq * D)


@pytest.mark.parametrize("T,offset,Hq,Hkv", [(1, 96, 6, 2), (1, 0, 4, 4), (33, 0, 4, 2),
                                             (9, 40, 6, 2)])
def test_attention_matches_fp64(oracle, T, offset, Hq, Hkv):
    # template: tests/test_nar.py:85-102 (bf16 attention vs fp64, rtol .004)
    rng = np.random.default_rng(62841 + T)
    cap = offset + T + 5
    q = bf(rng.normal(size=(T, Hq, 128)))
    keys = bf(rng.normal(size=(Hkv, cap, 128)))
    values = bf(rng.normal(size=(Hkv, cap, 128)))
    got = f(oracle.attention(q, keys, values, offset))
    ref = brute_attention(f(q), f(keys), f(values), offset)
    np.testing.assert_allclose(got, ref, rtol=0.008, atol=2e-3)
    # a wrong GQA map (h % Hkv) must be detected whenever it differs
    if Hq != Hkv:
        perm = np.array([h % Hkv for h in range(Hq)])
        alt = np.stack([brute_attention(f(q)[:, h:h + 1], f(keys)[perm[h]:perm[h] + 1],
                                        f(values)[perm[h]:perm[h] + 1], offset)
                        for h in range(Hq)], axis=1).reshape(T, -1)
        assert np.max(np.abs(alt - ref)) > 0.05


# ---- composition: golden vectors of the upstream torch model ----

def close(actual, expected, atol=2e-2, rtol=1e-2):
    return np.abs(actual - expected) <= atol + rtol * np.abs(expected)


def tiny_weights(g):
    import yuear
    w = yuear.random_weights(TINY, int(g["seed"]), float(g["std"]), float(g["norm_std"]))
    checksum = np.uint64(0)
    for name in sorted(w):
        checksum += np.uint64(int(w[name].astype(np.uint64).sum()))
    assert checksum == g["weight_checksum"], "weight generator drifted from the fixture"
    return w


def test_tiny_model_matches_torch_golden(oracle):
    g = np.load(os.path.join(GOLDEN, "tiny_model.npz"))
    model = oracle.Model(TINY, tiny_weights(g))
    cache = model.cache(16)
    logits = [model.prefill(g["prefix"].tolist(), cache)]
    logits += [model.step(int(t), cache) for t in g["steps"]]
    got = f(np.stack(logits))
    assert close(got, f(g["logits_bf16"])).all()
    assert close(got, g["logits_f32"]).all()
    assert (got.argmax(1) == f(g["logits_bf16"]).argmax(1)).all()


def test_tiny_golden_detects_a_dropped_qk_norm(oracle):
    # planted in the oracle: the same model without q/k RMSNorm must fail
    g = np.load(os.path.join(GOLDEN, "tiny_model.npz"))
    model = oracle.Model(dict(TINY, qk_norm=False), tiny_weights(g))
    cache = model.cache(16)
    got = f(model.prefill(g["prefix"].tolist(), cache))
    assert not close(got, f(g["logits_bf16"][0])).all()


def test_3b_layer_matches_torch_golden(oracle):
    import yuear
    from make_golden import LAYER
    g = np.load(os.path.join(GOLDEN, "layer_3072.npz"))
    seed, length = int(g["seed"]), int(g["length"])
    w = yuear.random_weights(LAYER, seed)
    kv = yuear.random_normal(seed, int(g["kv_stream"]), (2, 8, length - 1, 128))
    x = yuear.random_normal(seed, int(g["x_stream"]), (1, 3072))
    model = oracle.Model(LAYER, w)
    cache = model.cache(length)
    cache.keys(0)[:, :length - 1] = kv[0]
    cache.values(0)[:, :length - 1] = kv[1]
    cache.offset = length - 1
    got = f(model.layer(0, x, cache)[0])
    assert close(got, f(g["hidden_bf16"])).all()
    assert close(got, g["hidden_f32"], atol=5e-2).all()


def test_fp64_accumulation_mode_is_the_tighter_anchor(oracle):
    # the anchor used by the full-size fidelity tests: fp64 accumulation must
    # sit at least as close to the exact result as the default fp32 order
    rng = np.random.default_rng(8)
    x = bf(rng.normal(size=(3, 8192)))
    w = bf(rng.normal(size=(512, 8192)) * 0.02)
    exact = f(x).astype(np.float64) @ f(w).astype(np.float64).T
    y32 = f(oracle.linear(x, w))
    oracle.lib().oracle_set_accumulation(1)
    try:
        y64 = f(oracle.linear(x, w))
    finally:
        oracle.lib().oracle_set_accumulation(0)
    e32, e64 = np.abs(y32 - exact), np.abs(y64 - exact)
    assert e64.sum() <= e32.sum()
    # fp64 then one rounding: the nearest bf16 (within half a bf16 ulp)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
    assert (e64 <= 0.5 * ulp * (1 + 1e-6)).all()
