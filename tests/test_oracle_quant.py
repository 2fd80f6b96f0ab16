"""The oracle's affine group-64 quantized linear (ar.cpp:20-29, 306-312:
mx::quantized_matmul, transpose, group 64, bits 8 / 4, "affine") against what
the mathematics fixes (CPU):

- fp64 brute force over codes recovered through the byte view of the words
  (tests/quant_util.unpack_bytes), not the word shifts the oracle uses: a
  reversed nibble order or a wrong word index fails it;
- when every s * q + b is a bf16 value, the quantized linear equals the bf16
  linear over the dequantized matrix (up to fp32 summation order);
- all-zero codes leave the bias term alone (a dropped or doubled bias term
  fails it); codes that are one-hot per group pick single inputs;
- a quantized oracle model equals the bf16 oracle model over the
  dequantized weights when those are bf16 values (composition, phases).

The packing order itself (MLX quantize: code j of a word at bits bits * j)
is parity unpinned: MLX is absent and the reference holds no quantized
fixture.
"""
import numpy as np
import pytest

from conftest import TINY, assert_close_bf16
from quant_util import (LINEARS, bf, dequantize_f64, pack, quantize_model, random_quantized,
                        unpack_bytes)


def f(bits):
    import cpu_ref
    return cpu_ref.bf16_to_f32(bits)


@pytest.mark.parametrize("bits", [4, 8])
def test_pack_round_trips_through_the_byte_view(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, size=(7, 256))
    words = pack(codes, bits)
    assert words.shape == (7, 256 * bits // 32) and words.dtype == np.uint32
    np.testing.assert_array_equal(unpack_bytes(words, bits), codes)
    # element 0 sits in the low bits of word 0
    one = np.zeros((1, 64), np.int64)
    one[0, 0] = 1
    assert pack(one, bits)[0, 0] == 1
    one[0, 0], one[0, 1] = 0, 1
    assert pack(one, bits)[0, 0] == 1 << bits


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("k", [256, 3072])
def test_qlinear_matches_fp64(oracle, bits, k):
    rng = np.random.default_rng(k + bits)
    x = bf(rng.normal(size=(3, k)))
    w, s, b, _ = random_quantized(rng, 129, k, bits)
    codes = unpack_bytes(w, bits)
    ref = f(x).astype(np.float64) @ dequantize_f64(codes, s, b).T
    got = f(oracle.qlinear(x, w, s, b, bits))
    scale = np.abs(ref).max()
    err = np.abs(got - ref)
    assert (err <= 2.0 ** -8 * np.abs(ref) + 2.0 ** -12 * scale).all(), err.max()


@pytest.mark.parametrize("bits", [4, 8])
def test_qlinear_equals_linear_on_exact_dequantized_weights(oracle, bits):
    rng = np.random.default_rng(11 + bits)
    k, n = 512, 96
    levels = (1 << bits) - 1
    codes = rng.integers(0, levels + 1, size=(n, k))
    # power-of-two scales and biases on their grid: every s q + b is a bf16
    # value (at most 8 significant bits)
    e = rng.integers(-9, -5, size=(n, k // 64))
    s = bf(np.exp2(e).astype(np.float32))
    b = bf(-np.exp2(e) * (levels // 2))
    w = pack(codes, bits)
    deq = oracle.dequantize(w, s, b, bits)
    np.testing.assert_array_equal(f(deq).astype(np.float64), dequantize_f64(codes, s, b))
    x = bf(rng.normal(size=(4, k)))
    assert_close_bf16(oracle.qlinear(x, w, s, b, bits), oracle.linear(x, deq), exact_frac=0.9)


@pytest.mark.parametrize("bits", [4, 8])
def test_qlinear_bias_term_and_one_hot_codes(oracle, bits):
    rng = np.random.default_rng(5)
    k, n = 256, 8
    x = bf(rng.normal(size=(2, k)))
    s = bf(np.full((n, k // 64), 0.5))
    b = bf(rng.normal(size=(n, k // 64)))
    zero = pack(np.zeros((n, k), np.int64), bits)
    xs = f(x).astype(np.float64).reshape(2, k // 64, 64).sum(-1)
    ref = xs @ f(b).astype(np.float64).T
    got = f(oracle.qlinear(x, zero, s, b, bits))
    np.testing.assert_allclose(got, ref, rtol=2.0 ** -7, atol=1e-6)
    # zero biases, code 2 at column c of row r in every group: y = sum_g x[g*64 + c]
    codes = np.zeros((n, k), np.int64)
    for r in range(n):
        codes[r, (r * 5) % 64::64] = 2
    b0 = np.zeros_like(b)
    got = f(oracle.qlinear(x, pack(codes, bits), s, b0, bits))
    ref = np.stack([f(x).astype(np.float64)[:, (r * 5) % 64::64].sum(-1) for r in range(n)], -1)
    np.testing.assert_allclose(got, ref, rtol=2.0 ** -7, atol=1e-6)


def exact_quantized_model(weights, bits, seed):
    """Quantized weights whose dequantized values are bf16 numbers, and the
    bf16 weight dict of those values."""
    import cpu_ref
    rng = np.random.default_rng(seed)
    levels = (1 << bits) - 1
    q, deq = {}, {}
    for name, value in weights.items():
        base = name[:-len(".weight")]
        if base == "lm_head" or base.endswith(LINEARS):
            rows, k = value.shape
            codes = rng.integers(0, levels + 1, size=(rows, k))
            e = rng.integers(-10, -7, size=(rows, k // 64))
            s, b = bf(np.exp2(e).astype(np.float32)), bf(-np.exp2(e) * (levels // 2))
            q[name], q[base + ".scales"], q[base + ".biases"] = pack(codes, bits), s, b
            deq[name] = cpu_ref.dequantize(q[name], s, b, bits)
        else:
            q[name] = deq[name] = value
    return q, deq


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_model_composes_like_the_bf16_model(oracle, yuear_lib, bits):
    cfg = dict(TINY, vocab_size=184704)  # the YuE2 vocabulary: every phase's rows
    weights = yuear_lib.random_weights(dict(TINY), seed=3, norm_std=0.1)
    weights["model.embed_tokens.weight"] = bf(
        np.random.default_rng(1).normal(size=(cfg["vocab_size"], TINY["hidden_size"])) * 0.02)
    weights["lm_head.weight"] = np.zeros((cfg["vocab_size"], TINY["hidden_size"]), np.uint16)
    q, deq = exact_quantized_model(weights, bits, seed=bits)
    mq, md = oracle.Model(cfg, q, bits=bits), oracle.Model(cfg, deq)
    ids = [5, 151640, 77, 9]
    for phase in ("full", "abc", "semantic"):
        cq, cd = mq.cache(8), md.cache(8)
        lq, ld = mq.prefill(ids, cq, phase), md.prefill(ids, cd, phase)
        assert lq.shape == ld.shape == (mq.phase_size(phase),)
        assert_close_bf16(lq, ld, exact_frac=0.9)
        assert_close_bf16(mq.step(3, cq, phase), md.step(3, cd, phase), exact_frac=0.9)


def test_random_quantized_dict_has_the_reference_shapes(yuear_lib):
    weights = yuear_lib.random_weights(TINY, seed=1)
    for bits in (4, 8):
        q = quantize_model(weights, bits)
        H, F = TINY["hidden_size"], TINY["intermediate_size"]
        down = "model.layers.1.mlp.down_proj"
        assert q[down + ".weight"].shape == (H, F * bits // 32)
        assert q[down + ".weight"].dtype == np.uint32
        assert q[down + ".scales"].shape == q[down + ".biases"].shape == (H, F // 64)
        assert q["lm_head.scales"].shape == (TINY["vocab_size"], H // 64)
        assert q["model.embed_tokens.weight"].dtype == np.uint16
        assert "model.layers.0.input_layernorm.scales" not in q
