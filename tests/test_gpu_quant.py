"""Affine group-64 quantized linears ("8bit" / "4bit" precisions, ar.cpp:20-29,
209-214, 306-312) on the GPU against the oracle's quantized linear and model.

- op level: the quantized GEMV (batch 1-2, every prologue / epilogue, the
  input widths of the 3B and YuE2 layers and small ones) against
  oracle.qlinear, and the dequantization kernel bit for bit against
  oracle.dequantize;
- engine: prefill (MFMA GEMMs over the dequantized rows) and decode steps
  (the quantized GEMVs) of quantized tiny models against the quantized oracle
  model; batched sequences (dequantized rows, MFMA GEMV); the RANDOM source
  against host tensors quantized by the same quantizer; checkpoints of both
  precisions against host tensors, bit for bit.

Codes are drawn at random (tests/quant_util.py), so no converter is involved.
"""
import numpy as np
import pytest

from checkpoint_util import write_checkpoint
from conftest import TINY, assert_close_bf16
from quant_util import quantize_model, random_quantized

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-2, 1e-2  # logits tolerance of the decode path


@pytest.fixture(scope="module")
def torch():
    import torch as t
    t.cuda.init()
    return t


def dev(torch, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def host(torch, t):
    torch.cuda.synchronize()
    out = t.cpu().numpy()
    return out.view(np.uint16) if out.dtype == np.int16 else out


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


def f(b):
    import cpu_ref
    return cpu_ref.bf16_to_f32(b)


def group_words(scales, biases):
    return (scales.astype(np.uint32) | (biases.astype(np.uint32) << 16)).astype(np.uint32)


QGEMV_CASES = [  # (n, k, batch, norm, epilogue)
    (5120, 3072, 1, True, 0),     # fused QKV + input RMSNorm (3B)
    (3072, 3072, 1, False, 1),    # o_proj + residual
    (16384, 3072, 1, True, 2),    # gate/up interleaved + SwiGLU
    (3072, 8192, 1, False, 1),    # down + residual
    (83968, 3072, 1, True, 0),    # lm_head + final norm
    (5120, 3072, 2, True, 0),     # CFG pair
    (3072, 8192, 2, False, 1),
    (16384, 3072, 2, True, 2),
    (4096, 2048, 1, True, 0),     # YuE2 layer widths
    (12288, 2048, 2, True, 2),
    (2048, 6144, 1, False, 1),
    (1000, 256, 1, True, 0),      # short rows: 8 / 16 lanes per row, ragged n
    (96, 512, 2, False, 2),
    (200, 1024, 1, False, 0),
    (998, 4096, 2, True, 2),
]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n,k,batch,norm,epilogue", QGEMV_CASES)
def test_qgemv_matches_oracle(torch, yuear_lib, oracle, bits, n, k, batch, norm, epilogue):
    print(f"[qgemv] bits={bits} n={n} k={k} batch={batch} norm={norm} epi={epilogue}", flush=True)
    rng = np.random.default_rng(n + k + batch + bits)
    w, s, b, _ = random_quantized(rng, n, k, bits)
    x = bf(rng.normal(size=(batch, k)))
    g = bf(1 + rng.normal(size=k) * 0.1)
    out_n = n // 2 if epilogue == 2 else n
    y0 = bf(rng.normal(size=(batch, out_n)))
    h = oracle.rms_norm(x, g, 1e-5) if norm else x
    acc = oracle.qlinear(h, w, s, b, bits)
    if epilogue == 0:
        ref = acc
    elif epilogue == 1:
        ref = bf(f(y0) + f(acc))
    else:
        ref = oracle.silu_mul(acc[:, 0::2], acc[:, 1::2])
    dw, dsb, dx, dg = dev(torch, w), dev(torch, group_words(s, b)), dev(torch, x), dev(torch, g)
    dy = dev(torch, y0 if epilogue == 1 else np.zeros((batch, out_n), np.uint16))
    rc = yuear_lib.lib.yuear_op_qgemv(dw.data_ptr(), dsb.data_ptr(), bits, n, k, batch,
                                      dx.data_ptr(), k, dg.data_ptr() if norm else None, 1e-5,
                                      dy.data_ptr(), out_n, epilogue, None)
    assert rc == 0
    got = host(torch, dy)
    scale = max(np.abs(f(acc)).max(), np.abs(f(ref)).max())
    assert_close_bf16(got, ref, scale=scale, exact_frac=0.9)


def test_qgemv_rejects_unsupported_shapes(torch, yuear_lib):
    d = dev(torch, np.zeros(4096, np.uint32))
    y = dev(torch, np.zeros(64, np.uint16))
    for bits, k, batch in ((4, 96, 1), (3, 256, 1), (4, 256, 3), (8, 8256, 1)):
        rc = yuear_lib.lib.yuear_op_qgemv(d.data_ptr(), d.data_ptr(), bits, 8, k, batch,
                                          y.data_ptr(), k, None, 1e-5, y.data_ptr(), 8, 0, None)
        assert rc != 0, (bits, k, batch)
    # rows that would overlap: activation stride below k, output stride below n
    for xs, ys in ((256 - 8, 8), (256, 7)):
        rc = yuear_lib.lib.yuear_op_qgemv(d.data_ptr(), d.data_ptr(), 4, 8, 256, 2,
                                          y.data_ptr(), xs, None, 1e-5, y.data_ptr(), ys, 0, None)
        assert rc != 0, (xs, ys)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_is_bit_exact(torch, yuear_lib, oracle, bits):
    rng = np.random.default_rng(bits)
    n, k = 300, 3072
    w, s, b, _ = random_quantized(rng, n, k, bits)
    dw, dsb = dev(torch, w), dev(torch, group_words(s, b))
    out = dev(torch, np.zeros((n, k), np.uint16))
    assert yuear_lib.lib.yuear_op_dequantize(dw.data_ptr(), dsb.data_ptr(), bits, n, k,
                                             out.data_ptr(), None) == 0
    np.testing.assert_array_equal(host(torch, out), oracle.dequantize(w, s, b, bits))


def within(a, b, atol=ATOL, rtol=RTOL):
    return np.abs(f(a) - f(b)) <= atol + rtol * np.abs(f(b))


@pytest.fixture(scope="module", params=[4, 8])
def qtiny(request, yuear_lib, oracle):
    bits = request.param
    w = quantize_model(yuear_lib.random_weights(TINY, seed=21, norm_std=0.1), bits, seed=bits)
    return bits, yuear_lib.Engine(TINY, w, bits=bits), oracle.Model(TINY, w, bits=bits), w


def test_quantized_engine_prefill_and_steps_match_oracle(qtiny):
    bits, engine, model, _ = qtiny
    print(f"[quant engine] bits={bits}", flush=True)
    assert engine.bits == bits
    s = engine.session(1, 32)
    cache = model.cache(32)
    prefix, steps = [3, 17, 255, 1, 98, 400, 7], [12, 99, 300, 5, 511]
    got = [s.prefill(0, prefix)] + [s.step(t)[0] for t in steps]
    want = [model.prefill(prefix, cache)] + [model.step(t, cache) for t in steps]
    got, want = np.stack(got), np.stack(want)
    # prefill runs MFMA GEMMs over the dequantized rows, each weight rounded
    # to bf16 (up to 2^-9 relative), where the oracle sums the codes exactly;
    # the decode steps inherit that through the cache: the logits stay
    # within the decode path's tolerance (a few bf16 units of their scale)
    assert within(got, want).all()
    # greedy choice, gap-aware: where the argmax differs, the oracle's top two
    # logits are closer than the tolerance (random codes make near ties)
    pick = f(got).argmax(1)
    top = f(want).max(1)
    assert (f(want)[np.arange(len(pick)), pick] >= top - 2 * (ATOL + RTOL * np.abs(top))).all()


def test_quantized_decode_steps_match_oracle_on_its_cache(qtiny):
    """Each decode step (every projection and the lm_head on the quantized
    GEMV) from the oracle's own cache: within one bf16 unit at the logits'
    scale (2^-7 of max |logit|). The GEMV sums a piece's codes against the
    activations with the offset-128 pairs and folds the bias in per piece,
    the oracle per group (>= 99.8 % of GEMV outputs bit-identical, the rest
    one unit apart), and the attention sums keys in MFMA order; two layers
    carry such units to the logits."""
    bits, engine, model, _ = qtiny
    print(f"[quant steps] bits={bits}", flush=True)
    s = engine.session(1, 32)
    cache = model.cache(32)
    prefix = [3, 17, 255, 1, 98, 400, 7]
    model.prefill(prefix, cache)
    n = len(prefix)
    for t in (12, 99, 300, 5, 511):
        for layer in range(TINY["num_hidden_layers"]):
            s.write_kv(layer, 0, cache.keys(layer)[:, :n], cache.values(layer)[:, :n])
        got, want = s.step(t)[0], model.step(t, cache)
        n += 1
        err = np.abs(f(got) - f(want))
        assert (err <= 2.0 ** -7 * np.abs(f(want)).max()).all(), (t, err.max())


def test_quantized_engine_cfg_pair_and_batched_sequences(qtiny):
    bits, engine, model, _ = qtiny
    print(f"[quant batched] bits={bits}", flush=True)
    prefixes = [[2, 3, 4, 5], [6, 50, 7], [9], [100, 101, 102, 103, 104], [77, 1]]
    for branches in (2, 5):
        s = engine.session(branches, 16)
        caches = [model.cache(16) for _ in range(branches)]
        for bi in range(branches):
            got = s.prefill(bi, prefixes[bi])
            assert within(got, model.prefill(prefixes[bi], caches[bi])).all()
        toks = [10 + bi for bi in range(branches)]
        got = s.step(toks)
        for bi in range(branches):
            assert within(got[bi], model.step(toks[bi], caches[bi])).all(), (branches, bi)


def test_quantized_engine_rejects_bf16_linears(yuear_lib):
    w = yuear_lib.random_weights(TINY, seed=2)
    with pytest.raises(ValueError, match="Missing AR tensor|Incompatible AR tensor"):
        yuear_lib.Engine(TINY, w, bits=4)
    q = quantize_model(w, 8)
    with pytest.raises(ValueError, match="Incompatible AR tensor shape/dtype"):
        yuear_lib.Engine(TINY, q, bits=4)


@pytest.mark.parametrize("bits", [4, 8])
def test_random_source_quantizes_like_host_tensors(yuear_lib, bits):
    print(f"[quant random] bits={bits}", flush=True)
    w = yuear_lib.random_weights(TINY, seed=5, std=0.02, norm_std=0.1)
    a = yuear_lib.Engine(TINY, seed=5, std=0.02, norm_std=0.1, bits=bits)
    b = yuear_lib.Engine(TINY, yuear_lib.quantized_weights(w, bits), bits=bits)
    try:
        out = []
        for e in (a, b):
            s = e.session(1, 16)
            out.append([s.prefill(0, [4, 8, 15, 16])] + [s.step(t)[0] for t in (23, 42)])
            s.close()
        for x, y in zip(*out):
            np.testing.assert_array_equal(x, y)
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("bits,writer,pad_odd", [(4, "safetensors", False), (8, "raw", True)])
def test_quantized_checkpoint_matches_host_tensors(yuear_lib, tmp_path, bits, writer, pad_odd):
    print(f"[quant checkpoint] bits={bits} writer={writer}", flush=True)
    w = quantize_model(yuear_lib.random_weights(TINY, seed=13, norm_std=0.1), bits, seed=1)
    precision = f"{bits}bit"
    kw = {"pad_odd": True} if pad_odd else {}
    d = write_checkpoint(tmp_path / "ck", TINY, w, precision=precision, writer=writer, **kw)
    loaded = yuear_lib.Engine.load(str(d), precision)
    direct = yuear_lib.Engine(TINY, w, bits=bits)
    try:
        assert loaded.bits == bits
        out = []
        for e in (loaded, direct):
            s = e.session(1, 32)
            out.append([s.prefill(0, [5, 77, 301, 12])] + [s.step(t)[0] for t in (44, 500, 3)])
            s.close()
        for x, y in zip(*out):
            np.testing.assert_array_equal(x, y)
    finally:
        loaded.close()
        direct.close()
