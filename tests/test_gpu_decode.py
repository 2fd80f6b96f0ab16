"""Persistent decode step (one launch per token) and the fused QKV +
attention + o_proj layer launch against the per-op decode kernels on the GPU.

The persistent kernel repeats the per-op kernels' arithmetic operation for
operation, so the two paths must agree bit for bit: logits of every step,
every KV slot appended, positions; and through the sampler, the emitted
tokens. The per-op path itself is pinned against the oracle and the golden
vectors in test_gpu_engine.py / test_gpu_full.py; this file closes the chain
for the persistent path (ar.cpp:246-323 decode step, sampling.cpp:185-288
loop). Shapes cover both compiled hidden sizes, one and two branches, ragged
branch lengths, a single-split cache, a 33-split cache at KV ~4096 and the
semantic phase's odd logits row count (32769 rows, a ragged last task).
"""
import numpy as np
import pytest

from conftest import MODEL_3B, check_fidelity

pytestmark = pytest.mark.gpu

TWO_LAYER = dict(MODEL_3B, num_hidden_layers=2)
# the semantic phase reads the native codec rows [151852, 151852 + 32769)
TWO_LAYER_NATIVE = dict(TWO_LAYER, vocab_size=184704)
HIDDEN_2048 = dict(hidden_size=2048, intermediate_size=6144, num_hidden_layers=3,
                   num_attention_heads=16, num_key_value_heads=8, head_dim=128, vocab_size=8192,
                   max_position_embeddings=4096, rms_norm_eps=1e-6, rope_theta=1e6, qk_norm=True)


@pytest.fixture(scope="module")
def engine(yuear_lib):
    e = yuear_lib.Engine(TWO_LAYER, None, seed=11)
    yield e
    e.close()


def run(engine, path, branches, capacity, prompts, steps, phase="full"):
    print(f"[decode] path={path} branches={branches} cap={capacity} "
          f"prompts={[len(p) for p in prompts]} steps={len(steps)} phase={phase}", flush=True)
    s = engine.session(branches, capacity, phase)
    s.decode_path = path
    assert s.decode_path == path
    for b, p in enumerate(prompts):
        s.prefill(b, p)
    logits = np.stack([s.step(t) for t in steps])
    pos = [s.position(b) for b in range(branches)]
    layers = engine.config["num_hidden_layers"]
    kv = [s.read_kv(layer, b, pos[b]) for layer in range(layers) for b in range(branches)]
    s.close()
    return logits, kv, pos


def assert_same(a, b):
    la, kva, pa = a
    lb, kvb, pb = b
    assert pa == pb
    np.testing.assert_array_equal(la, lb)
    for (ka, va), (kb, vb) in zip(kva, kvb):
        np.testing.assert_array_equal(ka, kb)
        np.testing.assert_array_equal(va, vb)


@pytest.mark.parametrize("branches,capacity,lengths,n_steps", [
    (1, 64, [5], 6),
    (1, 20, [1], 18),           # one split; fills the cache to its last slot
    (2, 700, [513, 200], 4),    # ragged branches
    (1, 4200, [4090], 3),       # 33 splits around KV 4096
])
def test_persistent_step_matches_per_op_kernels_bitwise(engine, branches, capacity, lengths,
                                                        n_steps):
    rng = np.random.default_rng(capacity + branches)
    V = engine.config["vocab_size"]
    prompts = [rng.integers(0, V, size=n).tolist() for n in lengths]
    steps = [rng.integers(0, V, size=branches).tolist() for _ in range(n_steps)]
    a = run(engine, "kernels", branches, capacity, prompts, steps)
    b = run(engine, "persistent", branches, capacity, prompts, steps)
    assert_same(a, b)
    assert np.isfinite(a[0].view(np.uint16).astype(np.float32)).all()


@pytest.mark.parametrize("branches,capacity,lengths,n_steps", [
    (1, 64, [5], 6),
    (1, 20, [1], 18),           # one split; fills the cache to its last slot
    (2, 700, [513, 200], 4),    # ragged branches
    (1, 4200, [4090], 3),       # 33 splits around KV 4096
])
def test_fused_layer_matches_per_op_kernels_bitwise(engine, branches, capacity, lengths,
                                                    n_steps):
    rng = np.random.default_rng(capacity + 7 * branches)
    V = engine.config["vocab_size"]
    prompts = [rng.integers(0, V, size=n).tolist() for n in lengths]
    steps = [rng.integers(0, V, size=branches).tolist() for _ in range(n_steps)]
    assert_same(run(engine, "kernels", branches, capacity, prompts, steps),
                run(engine, "fused", branches, capacity, prompts, steps))


@pytest.mark.parametrize("config", ["tiny", "hidden_2048"])
def test_fused_layer_other_shapes(yuear_lib, config):
    from conftest import TINY
    cfg = {"tiny": TINY, "hidden_2048": HIDDEN_2048}[config]
    e = yuear_lib.Engine(cfg, None, seed=21)
    try:
        V = cfg["vocab_size"]
        rng = np.random.default_rng(6)
        prompts = [rng.integers(0, V, size=n).tolist() for n in (9, 4)]
        steps = [rng.integers(0, V, size=2).tolist() for _ in range(5)]
        cap = min(64, cfg["max_position_embeddings"])
        assert_same(run(e, "kernels", 2, cap, prompts, steps), run(e, "fused", 2, cap, prompts, steps))
        assert_same(run(e, "kernels", 1, cap, prompts[:1], [s[:1] for s in steps]),
                    run(e, "fused", 1, cap, prompts[:1], [s[:1] for s in steps]))
    finally:
        e.close()


def test_fused_path_after_persistent_steps(engine):
    # Steps of the persistent path do not advance the fused path's step
    # counter; switching back must not let words of the last fused step pass
    # for fresh ones. Interleave the paths and compare with the per-op path.
    rng = np.random.default_rng(14)
    prompt = rng.integers(0, 83968, size=21).tolist()
    toks = rng.integers(0, 83968, size=6).tolist()
    ref = engine.session(1, 64)
    ref.decode_path = "kernels"
    ref.prefill(0, prompt)
    want = [ref.step(t) for t in toks]
    ref.close()
    s = engine.session(1, 64)
    s.decode_path = "fused"
    s.prefill(0, prompt)
    got = []
    for i, t in enumerate(toks):
        s.decode_path = ("fused", "persistent")[i % 2]
        got.append(s.step(t))
    s.close()
    np.testing.assert_array_equal(np.stack(got), np.stack(want))


def test_fused_expired_wait_is_reported(engine, monkeypatch):
    # A wait bound of 0 makes every wait that is not satisfied on its first
    # read give up (o_proj workgroups start while the attention still runs);
    # the kernel runs to its end and the host reports the expired wait.
    monkeypatch.setenv("YUEAR_FUSED_WAIT_US", "0")
    s = engine.session(1, 32)
    s.decode_path = "fused"
    s.prefill(0, [1, 2, 3])
    with pytest.raises(RuntimeError, match="dependency wait expired"):
        s.step(4)
    s.close()
    monkeypatch.delenv("YUEAR_FUSED_WAIT_US")
    a = engine.session(1, 32)
    a.decode_path = "fused"
    a.prefill(0, [1, 2, 3])
    b = engine.session(1, 32)
    b.prefill(0, [1, 2, 3])
    np.testing.assert_array_equal(a.step(4), b.step(4))
    a.close()
    b.close()


def test_semantic_phase_odd_row_count(yuear_lib):
    e = yuear_lib.Engine(TWO_LAYER_NATIVE, None, seed=5)
    try:
        rng = np.random.default_rng(3)
        prompts = [rng.integers(0, 184704, size=40).tolist()]
        steps = [[int(t)] for t in rng.integers(151853, 151853 + 32768, size=3)]
        a = run(e, "kernels", 1, 64, prompts, steps, phase="semantic")
        b = run(e, "persistent", 1, 64, prompts, steps, phase="semantic")
        assert a[0].shape[-1] == 32769
        assert_same(a, b)
    finally:
        e.close()


def test_hidden_2048_two_branches(yuear_lib):
    e = yuear_lib.Engine(HIDDEN_2048, None, seed=9)
    try:
        rng = np.random.default_rng(4)
        prompts = [rng.integers(0, 8192, size=n).tolist() for n in (100, 37)]
        steps = [rng.integers(0, 8192, size=2).tolist() for _ in range(5)]
        assert_same(run(e, "kernels", 2, 300, prompts, steps),
                    run(e, "persistent", 2, 300, prompts, steps))
    finally:
        e.close()


def test_unsupported_shape_keeps_per_op_path(yuear_lib):
    from conftest import TINY
    e = yuear_lib.Engine(TINY, None, seed=1)
    try:
        s = e.session(1, 16)
        assert s.decode_path == "kernels"
        with pytest.raises(ValueError, match="persistent decode step is not available"):
            s.decode_path = "persistent"
        s.decode_path = "fused"
        s.close()
        s = e.session(3, 16)  # more than two branches: per-op kernels
        assert s.decode_path == "kernels"
        with pytest.raises(ValueError, match="fused decode layer is not available"):
            s.decode_path = "fused"
        s.close()
    finally:
        e.close()


GREEDY = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0, penalty_window=50,
              min_tokens=0, max_tokens=64)
SAMPLED = dict(temperature=0.9, top_p=0.9, top_k=40, repetition_penalty=1.1, penalty_window=20,
               min_tokens=0, max_tokens=64)


@pytest.mark.parametrize("sampling", [GREEDY, SAMPLED], ids=["greedy", "sampled"])
def test_device_loop_tokens_agree(engine, sampling):
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, 83968, size=77).tolist()
    out = {}
    for path in ("kernels", "persistent", "fused"):
        s = engine.session(1, 256)
        s.decode_path = path
        last = s.prefill(0, prompt)
        ms, tokens = s.time_generate(sampling, 1234, 24, reset=True)
        out[path] = (tokens, s.position(0), s.read_kv(1, 0, s.position(0)))
        s.close()
        assert ms > 0 and last.shape == (83968,)
    for path in ("persistent", "fused"):
        assert out["kernels"][0] == out[path][0]
        assert out["kernels"][1] == out[path][1]
        np.testing.assert_array_equal(out["kernels"][2][0], out[path][2][0])


def test_generate_tokens_on_persistent_path(engine, monkeypatch):
    rng = np.random.default_rng(9)
    prefix = rng.integers(0, 83968, size=50).tolist()
    sampling = dict(SAMPLED, max_tokens=20)
    monkeypatch.setenv("YUEAR_DECODE", "kernels")
    want, _, _ = engine.generate_tokens(prefix, sampling, 77)
    monkeypatch.setenv("YUEAR_DECODE", "persistent")
    got, timing, _ = engine.generate_tokens(prefix, sampling, 77)
    assert got == want and timing["execution"] == "hip_graph"


def test_decode_step_timing_restores_positions(engine):
    rng = np.random.default_rng(10)
    prompt = rng.integers(0, 83968, size=30).tolist()
    tok = int(rng.integers(0, 83968))
    s = engine.session(1, 64)
    s.decode_path = "persistent"
    s.prefill(0, prompt)
    ms = s.time_kernel("decode_step", 5)
    assert ms > 0 and s.position(0) == 30
    got = s.step(tok)
    s.close()
    r = engine.session(1, 64)
    r.prefill(0, prompt)
    np.testing.assert_array_equal(got, r.step(tok))
    r.close()


def test_expired_wait_is_reported(engine, monkeypatch):
    # A spin limit of 0 makes every dependency wait that is not already
    # satisfied on its first poll give up: the kernel still runs to its end
    # (all reads stay in bounds whatever the activations hold) and the host
    # must report the expired wait instead of returning the logits.
    monkeypatch.setenv("YUEAR_DECODE_SPIN_LIMIT", "0")
    s = engine.session(1, 32)
    s.decode_path = "persistent"
    s.prefill(0, [1, 2, 3])
    with pytest.raises(RuntimeError, match="dependency wait expired"):
        s.step(4)
    s.close()
    monkeypatch.delenv("YUEAR_DECODE_SPIN_LIMIT")
    a = engine.session(1, 32)
    a.decode_path = "persistent"
    a.prefill(0, [1, 2, 3])
    b = engine.session(1, 32)
    b.prefill(0, [1, 2, 3])
    np.testing.assert_array_equal(a.step(4), b.step(4))
    a.close()
    b.close()


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
