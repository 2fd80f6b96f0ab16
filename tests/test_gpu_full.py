"""The BASELINE 3B decoder at full size on the GPU vs the oracle.

28 layers, hidden 3072, 24/8 heads, FFN 8192, vocab 83968, N(0, 0.02)
weights with unit norm gains (the bench's model). The oracle's CPU decode step
is ~1 s at this size, so these tests compare a few teacher-forced steps:
after a short prefill, and at KV length 4096 (the benchmark's metric point)
with the GPU's own cache copied to the oracle so both sides decode the same
state.
"""
import numpy as np
import pytest

from conftest import BASE_3B, ulps_bf16

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-2, 1e-2


def f(b):
    import cpu_ref
    return cpu_ref.bf16_to_f32(b)


@pytest.fixture(scope="module")
def pair(yuear_lib, oracle):
    w = yuear_lib.random_weights(BASE_3B, 20251201)
    engine = yuear_lib.Engine(BASE_3B, w)
    model = oracle.Model(BASE_3B, w)
    yield engine, model
    engine.close()


def check_logits(got, want):
    d = np.abs(f(got) - f(want))
    assert (d <= ATOL + RTOL * np.abs(f(want))).all(), d.max()
    assert f(got).argmax() == f(want).argmax() or \
        np.sort(f(want))[-1] - np.sort(f(want))[-2] < 2 * ATOL
    return ulps_bf16(got, want)


def test_full_model_short_prefill_and_steps(pair):
    engine, model = pair
    rng = np.random.default_rng(1)
    prefix = rng.integers(0, 83968, size=24).tolist()
    s = engine.session(1, 64)
    cache = model.cache(64)
    check_logits(s.prefill(0, prefix), model.prefill(prefix, cache))
    for t in rng.integers(0, 83968, size=2).tolist():
        check_logits(s.step(t)[0], model.step(t, cache))
    s.close()


def test_full_model_decode_at_kv_4096(pair):
    engine, model = pair
    rng = np.random.default_rng(2)
    prefix = rng.integers(0, 83968, size=4095).tolist()
    s = engine.session(1, 4100)
    s.prefill(0, prefix)
    cache = model.cache(4100)
    for layer in range(BASE_3B["num_hidden_layers"]):
        k, v = s.read_kv(layer, 0, 4095)
        cache.keys(layer)[:, :4095] = k
        cache.values(layer)[:, :4095] = v
    cache.offset = 4095
    token = int(rng.integers(0, 83968))
    check_logits(s.step(token)[0], model.step(token, cache))  # L = 4096
    k, v = s.read_kv(0, 0, 4096)  # the appended slot equals the oracle's
    assert ulps_bf16(k[:, 4095], cache.keys(0)[:, 4095]).max() <= 1
    s.close()
