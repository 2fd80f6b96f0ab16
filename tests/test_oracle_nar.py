"""The oracle's acoustic-model attention (nar_attention.cpp:63-270: the
non-causal kernel lyra_nar_precise_attention, and the causal conditioning
prefill of nar.cpp:176) against what the mathematics fixes (CPU): fp64
brute force over every (batch, head, query) with grouped kv heads; invariance
under a joint permutation of the keys and values (a transposed operand or a
wrong key index fails it); the causal form equals the AR prefill attention
(ar.cpp:284-291) on the same tensors; equal keys give the mean of V.
"""
import numpy as np
import pytest

from conftest import assert_close_bf16


def f(b):
    import cpu_ref
    return cpu_ref.bf16_to_f32(b)


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


def fp64_attention(q, k, v, causal):
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    qf, kf, vf = (f(a).astype(np.float64) for a in (q, k, v))
    out = np.empty((B, Hq, Lq, D))
    for h in range(Hq):
        g = h // (Hq // Hkv)
        s = np.einsum("bqd,bkd->bqk", qf[:, h], kf[:, g]) / np.sqrt(D)
        if causal:
            s = np.where(np.arange(Lk)[None, None, :] > np.arange(Lq)[None, :, None], -np.inf, s)
        p = np.exp(s - s.max(-1, keepdims=True))
        out[:, h] = np.einsum("bqk,bkd->bqd", p / p.sum(-1, keepdims=True), vf[:, g])
    return out


@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,causal", [
    (1, 4, 2, 37, 300, False), (2, 6, 2, 9, 65, False), (1, 2, 1, 70, 70, True)])
def test_nar_attention_matches_fp64(oracle, B, Hq, Hkv, Lq, Lk, causal):
    rng = np.random.default_rng(Lq + Lk)
    q = bf(rng.normal(size=(B, Hq, Lq, 128)))
    k = bf(rng.normal(size=(B, Hkv, Lk, 128)))
    v = bf(rng.normal(size=(B, Hkv, Lk, 128)))
    ref = fp64_attention(q, k, v, causal)
    got = f(oracle.nar_attention(q, k, v, causal))
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 2e-2)) < 1e-2


def test_nar_attention_key_permutation_invariance(oracle):
    rng = np.random.default_rng(3)
    q = bf(rng.normal(size=(1, 4, 20, 128)))
    k = bf(rng.normal(size=(1, 2, 150, 128)))
    v = bf(rng.normal(size=(1, 2, 150, 128)))
    perm = rng.permutation(150)
    a = oracle.nar_attention(q, k, v)
    b = oracle.nar_attention(q, k[:, :, perm], v[:, :, perm])
    assert_close_bf16(a, b, exact_frac=0.9)
    # permuting the keys alone is not an invariance: it changes the output
    assert np.mean(oracle.nar_attention(q, k[:, :, perm], v) == a) < 0.2


def test_nar_causal_equals_ar_prefill_attention(oracle):
    rng = np.random.default_rng(5)
    T, Hq, Hkv = 40, 4, 2
    q = bf(rng.normal(size=(1, Hq, T, 128)))
    k = bf(rng.normal(size=(1, Hkv, T, 128)))
    v = bf(rng.normal(size=(1, Hkv, T, 128)))
    nar = oracle.nar_attention(q, k, v, causal=True)[0]            # [Hq][T][D]
    ar = oracle.attention(np.ascontiguousarray(q[0].transpose(1, 0, 2)), k[0], v[0], 0)
    assert_close_bf16(nar, ar.reshape(T, Hq, 128).transpose(1, 0, 2), exact_frac=0.9)


def test_nar_attention_equal_keys_give_the_mean_of_v(oracle):
    rng = np.random.default_rng(9)
    q = bf(rng.normal(size=(1, 2, 5, 128)))
    k = np.repeat(bf(rng.normal(size=(1, 1, 1, 128))), 33, axis=2)
    v = bf(rng.normal(size=(1, 1, 33, 128)))
    got = f(oracle.nar_attention(q, k, v))
    mean = f(v).astype(np.float64).mean(2, keepdims=True)
    np.testing.assert_allclose(got, np.broadcast_to(mean, got.shape), rtol=2 ** -7, atol=1e-6)
