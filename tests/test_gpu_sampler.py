"""Device sampler vs the oracle: identical tokens on identical logits.

The sampler (CFG merge, distribution(), draw) is integer/ordering logic plus
fp32 arithmetic whose every step is defined on both sides with the same
operations (portable exp/log, sequential sums in sorted order, Philox
uniforms), so the drawn token must be bit-identical to the oracle's
(the acceptance bar: "a bit-exact sampled token stream when both sides are fed
identical uniform draws").
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MUSIC_END, CODEC_OFFSET = 151852, 151853


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


def head_engine(yuear, vocab):
    cfg = dict(hidden_size=64, intermediate_size=64, num_hidden_layers=1, num_attention_heads=1,
               num_key_value_heads=1, head_dim=128, vocab_size=vocab,
               max_position_embeddings=4096, rms_norm_eps=1e-5, rope_theta=5e5)
    return yuear.Engine(cfg, seed=1)


@pytest.fixture(scope="module")
def engine_83968(yuear_lib):
    return head_engine(yuear_lib, 83968)


@pytest.fixture(scope="module")
def engine_yue2(yuear_lib):
    return head_engine(yuear_lib, 184704)


def oracle_token(oracle, logits, sampling, seed, step, history, phase, cfg=1.0, legacy=False):
    x = logits[0] if cfg == 1.0 else oracle.guided_logits(logits[0], logits[1], cfg)
    s = oracle.sampling_struct(**sampling)
    scores = oracle.distribution(x, s, history, step, phase, legacy)
    local = oracle.draw(scores, sampling["temperature"], seed, step)
    return oracle.lib().oracle_local_to_native(local, oracle.PHASES[phase])


def logits_for(rng, kind, branches, n):
    if kind == "normal":
        x = rng.normal(size=(branches, n)) * 2.5
    elif kind == "ties":  # heavy ties at the top-k / nucleus cut
        x = np.round(rng.normal(size=(branches, n)) * 2) / 2
    elif kind == "equal":  # every row tied: the candidate lists overflow LDS
        x = np.full((branches, n), 1.25)
    elif kind == "integers":  # ~300 rows tied at the 100th largest (4.0)
        x = np.round(rng.normal(size=(branches, n)) * 1.3)
    elif kind == "peaked":
        x = rng.normal(size=(branches, n))
        x[:, rng.integers(0, n, 3)] += 12
    else:  # flat: top-p needs many survivors
        x = rng.normal(size=(branches, n)) * 0.05
    return bf(x)


CASES = [
    # name, sampling overrides, branches/cfg, phase, logits kind
    ("greedy", dict(temperature=0, top_k=1, top_p=1), 1, 1.0, "full", "normal"),
    ("greedy-ties", dict(temperature=0, top_k=1, top_p=1), 1, 1.0, "full", "ties"),
    ("cfg-pair", dict(temperature=1.0, top_k=50, top_p=0.93), 2, 1.5, "full", "normal"),
    ("cfg-pair-ties", dict(temperature=1.0, top_k=50, top_p=0.93), 2, 1.5, "full", "ties"),
    ("topk-only", dict(temperature=0.7, top_k=20, top_p=1.0), 1, 1.0, "full", "normal"),
    ("topp-flat", dict(temperature=1.0, top_k=5000, top_p=0.5), 1, 1.0, "full", "flat"),
    ("all-vocab", dict(temperature=1.3, top_k=100000, top_p=1.0), 1, 1.0, "full", "normal"),
    ("peaked", dict(temperature=1.0, top_k=100, top_p=0.95), 1, 1.0, "full", "peaked"),
    # 257-512 survivors: the network sort in LDS
    ("topk-400", dict(temperature=1.0, top_k=400, top_p=0.9), 1, 1.0, "full", "normal"),
    # 1025-4096 survivors: the LDS sort of the rows gathered after the first digit
    ("topk-2000-cfg", dict(temperature=0.8, top_k=2000, top_p=0.8), 2, 1.5, "full", "normal"),
    # top k in the split form's range: every row tied (the last workgroup
    # falls back to the one-workgroup algorithm over all rows), and ~300
    # rows at or above the cut (the merge's digit passes and network sort)
    ("split-all-equal", dict(temperature=1.0, top_k=50, top_p=0.9), 1, 1.0, "full", "equal"),
    ("split-ties-k100", dict(temperature=1.0, top_k=100, top_p=0.97), 1, 1.0, "full", "integers"),
]


@pytest.mark.parametrize("name,over,branches,cfg,phase,kind", CASES, ids=[c[0] for c in CASES])
def test_sampler_bit_exact_vs_oracle(engine_83968, oracle, name, over, branches, cfg, phase,
                                     kind):
    rng = np.random.default_rng(len(name) * 977)
    sampling = dict(temperature=1.0, top_p=0.95, top_k=100, repetition_penalty=1.0,
                    penalty_window=50, min_tokens=0, max_tokens=9000)
    sampling.update(over)
    session = engine_83968.session(branches, 64, phase)
    for trial in range(12):
        logits = logits_for(rng, kind, branches, 83968)
        session.write_logits(logits)
        seed, step = int(rng.integers(0, 2**62)), int(rng.integers(0, 5000))
        got = session.sample(sampling, seed, step, cfg_scale=cfg)
        want = oracle_token(oracle, logits, sampling, seed, step, [], phase, cfg)
        assert got == want, (name, trial, got, want)
    session.close()


def test_sampler_penalty_and_min_tokens_semantic(engine_yue2, oracle):
    rng = np.random.default_rng(5)
    sampling = dict(temperature=1.0, top_p=0.95, top_k=100, repetition_penalty=1.2,
                    penalty_window=50, min_tokens=200, max_tokens=9000)  # semantic defaults
    session = engine_yue2.session(1, 64, "semantic")
    n = session.vocab
    assert n == 32769
    for trial in range(16):
        x = rng.normal(size=(1, n)) * 2
        hist = [CODEC_OFFSET + int(t) for t in rng.integers(0, 40, size=int(rng.integers(0, 90)))]
        x[0, [h - MUSIC_END for h in hist[-10:]]] += 3  # make the penalty matter
        x[0, 0] += 6 * (trial % 2)                       # end row high on odd trials
        logits = bf(x)
        session.write_logits(logits)
        step = len(hist) + (0 if trial % 4 < 2 else 300)  # before / after min_tokens
        seed = int(rng.integers(0, 2**62))
        got = session.sample(sampling, seed, step, history=hist)
        want = oracle_token(oracle, logits, sampling, seed, step, hist, "semantic")
        assert got == want, (trial, got, want)
    session.close()


@pytest.mark.parametrize("top_k,top_p", [(100, 0.95), (20, 1.0), (5000, 0.9)])
def test_sampler_end_row_both_penalised_and_masked(engine_yue2, oracle, top_k, top_p):
    # the end token inside the penalty window while min_tokens still masks
    # it: the row is special twice over (masked, then penalised: -inf either
    # way) and must be replaced once in the scores and their counts
    rng = np.random.default_rng(11 + top_k)
    sampling = dict(temperature=1.0, top_p=top_p, top_k=top_k, repetition_penalty=1.2,
                    penalty_window=50, min_tokens=200, max_tokens=9000)
    session = engine_yue2.session(1, 64, "semantic")
    n = session.vocab
    for trial in range(12):
        x = rng.normal(size=(1, n)) * 2
        hist = [CODEC_OFFSET + int(t) for t in rng.integers(0, 40, size=60)]
        for at in rng.integers(10, 60, size=1 + trial % 3):
            hist[int(at)] = MUSIC_END
        x[0, 0] += 8  # the end row would lead if it were not masked
        logits = bf(x)
        session.write_logits(logits)
        step = 100 if trial % 3 else 250  # masked, masked, unmasked
        seed = int(rng.integers(0, 2**62))
        got = session.sample(sampling, seed, step, history=hist)
        want = oracle_token(oracle, logits, sampling, seed, step, hist, "semantic")
        assert got == want, (trial, got, want)
        if step < 200:
            assert got != MUSIC_END
    session.close()


EOD, ABC_END = 151643, 151848


@pytest.mark.parametrize("temperature,top_k,top_p,branches,cfg", [
    (1.0, 30, 0.9, 1, 1.0),   # the ABC defaults
    (0.8, 100, 1.0, 2, 1.5),  # CFG pair, top k only
    (0.0, 1, 1.0, 1, 1.0),    # greedy
])
def test_sampler_abc_phase_tail_rows(engine_yue2, oracle, temperature, top_k, top_p, branches,
                                     cfg):
    # 151644 local rows: the last 8-row chunk is partial (rows 151640-151643)
    # and its last row is the end row (ABC_END), masked before min_tokens and
    # here also inside the penalty window
    rng = np.random.default_rng(31 + top_k)
    sampling = dict(temperature=temperature, top_p=top_p, top_k=top_k, repetition_penalty=1.3,
                    penalty_window=50, min_tokens=100, max_tokens=9000)
    session = engine_yue2.session(branches, 64, "abc")
    n = session.vocab
    assert n == EOD + 1
    for trial in range(9):
        x = rng.normal(size=(branches, n)) * 2
        hist = [int(t) for t in rng.integers(n - 200, n - 1, size=60)]
        if trial % 3 != 2:
            hist[-1 - trial] = ABC_END            # the end row penalised too
        x[:, [t for t in hist[-50:] if t < n - 1]] += 4
        x[:, n - 1] += 9                           # the end row would lead
        x[:, n - 4:n - 1] += 5 * (trial % 2)       # the other tail rows lead next
        logits = bf(x)
        session.write_logits(logits)
        step = 40 if trial % 3 else 150            # masked, masked, unmasked
        seed = int(rng.integers(0, 2**62))
        got = session.sample(sampling, seed, step, history=hist, cfg_scale=cfg)
        want = oracle_token(oracle, logits, sampling, seed, step, hist, "abc", cfg)
        assert got == want, (trial, got, want)
        if step < 100:
            assert got != ABC_END
    session.close()


@pytest.mark.parametrize("branches,cfg", [(1, 1.0), (2, 1.5)])
def test_greedy_with_penalty_and_end_mask(engine_yue2, oracle, branches, cfg):
    # the greedy path rescored only the penalised / masked rows: odd phase
    # size (32769) exercises the padded rows and the scalar tail
    rng = np.random.default_rng(7 + branches)
    sampling = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.3,
                    penalty_window=20, min_tokens=50, max_tokens=9000)
    session = engine_yue2.session(branches, 64, "semantic")
    n = session.vocab
    for trial in range(16):
        x = rng.normal(size=(branches, n))
        hist = [CODEC_OFFSET + int(t) for t in rng.integers(0, 30, size=40)]
        x[:, [h - MUSIC_END for h in hist[-20:]]] += 4      # penalised rows lead
        x[:, 0] += 5 * (trial % 2)                          # end row leads on odd trials
        x[:, n - 1] += 3 * (trial % 3 == 0)                 # the tail row
        logits = bf(x)
        session.write_logits(logits)
        step = 10 if trial % 4 < 2 else 60                  # masked / unmasked end row
        got = session.sample(sampling, 0, step, history=hist, cfg_scale=cfg)
        want = oracle_token(oracle, logits, sampling, 0, step, hist, "semantic", cfg)
        assert got == want, (trial, got, want)
    session.close()


def test_sampler_legacy_off_bf16_mode(engine_yue2, oracle):
    rng = np.random.default_rng(6)
    sampling = dict(temperature=1.0, top_p=0.9, top_k=30, repetition_penalty=1.005,
                    penalty_window=100, min_tokens=0, max_tokens=4096)
    session = engine_yue2.session(1, 64, "semantic")
    for trial in range(8):
        logits = bf(rng.normal(size=(1, session.vocab)) * 2)
        session.write_logits(logits)
        hist = [CODEC_OFFSET + int(t) for t in rng.integers(0, 50, size=30)]
        seed = int(rng.integers(0, 2**62))
        got = session.sample(sampling, seed, 31, history=hist, legacy_off=True)
        want = oracle_token(oracle, logits, sampling, seed, 31, hist, "semantic", legacy=True)
        assert got == want, (trial, got, want)
    session.close()


@pytest.fixture(scope="module")
def engine_4096(yuear_lib):
    return head_engine(yuear_lib, 4096)


# (engine, phase, top_k, temperature): the split form serves more than 8192
# rows at top k <= 128 and greedy; the one-workgroup form the rest.
LEGACY_OFF_FORMS = {
    "split-sampled": ("yue2", "semantic", 30, 1.0),
    "one-wg-sampled": ("yue2", "semantic", 200, 1.0),
    "split-greedy": ("yue2", "semantic", 1, 0.0),
    "one-wg-greedy": ("4096", "full", 1, 0.0),
}


def _local(phase, native):
    return native - MUSIC_END if phase == "semantic" else native


@pytest.mark.parametrize("penalty", [1.005, 1.2])
@pytest.mark.parametrize("form", sorted(LEGACY_OFF_FORMS))
def test_sampler_legacy_off_penalised_rows_lead(engine_yue2, engine_4096, oracle, form, penalty):
    # legacy-off (bf16) scores with the penalised history rows in the top k:
    # alpha = pow(p, count) is cast to bf16 before it scales a score
    # (sampling.cpp:67-70); with p = 1.005 that is 1.0078125, not 1.005
    which, phase, top_k, temperature = LEGACY_OFF_FORMS[form]
    engine = engine_yue2 if which == "yue2" else engine_4096
    rng = np.random.default_rng(int(penalty * 1000) + top_k)
    sampling = dict(temperature=temperature, top_p=0.95, top_k=top_k,
                    repetition_penalty=penalty, penalty_window=50, min_tokens=0, max_tokens=9000)
    session = engine.session(1, 64, phase)
    n = session.vocab
    base = CODEC_OFFSET if phase == "semantic" else 100
    for trial in range(12):
        x = rng.normal(size=(1, n)) * 2
        hist = [base + int(t) for t in rng.integers(0, 40, size=int(rng.integers(20, 60)))]
        x[0, [_local(phase, h) for h in hist[-50:]]] += 3  # penalised rows lead
        logits = bf(x)
        session.write_logits(logits)
        seed = int(rng.integers(0, 2**62))
        got = session.sample(sampling, seed, len(hist), history=hist, legacy_off=True)
        want = oracle_token(oracle, logits, sampling, seed, len(hist), hist, phase, legacy=True)
        assert got == want, (form, trial, got, want)
    if penalty == 1.005:
        # a penalised row at 7.0 against an unpenalised row at 6.9375 with a
        # lower index: bf16(7 / bf16(1.005)) = 6.9375 ties it (the lower
        # index wins, or the draw splits them evenly), while 7 / 1.005 in
        # fp32 would round to 6.96875 and always win
        u, pen = base + 4, base + 8
        x = rng.normal(size=(1, n)) * 0.5
        x[0, _local(phase, u)] = 6.9375
        x[0, _local(phase, pen)] = 7.0
        logits = bf(x)
        session.write_logits(logits)
        cold = dict(sampling, temperature=0.001 if temperature else 0.0)
        picks = set()
        for trial in range(12):
            seed = int(rng.integers(0, 2**62))
            got = session.sample(cold, seed, 1, history=[pen], legacy_off=True)
            want = oracle_token(oracle, logits, cold, seed, 1, [pen], phase, legacy=True)
            assert got == want, (form, "near tie", trial, got, want)
            picks.add(want)
        assert u in picks  # the case separates bf16 alpha from fp32 alpha
    session.close()


def test_sampler_known_answers_on_device(engine_yue2):
    # test_sampling.py:37-49 restated through the device sampler: only the
    # surviving rows can ever be drawn.
    session = engine_yue2.session(1, 64, "semantic")
    n = session.vocab
    base = np.full((1, n), -20.0, np.float32)
    base[0, 1:5] = [5, 4, 4, 3]
    session.write_logits(bf(base))
    drawn = {session.sample(dict(temperature=1.0, top_k=2, top_p=1.0, repetition_penalty=1.0,
                                 min_tokens=0, max_tokens=100), seed, 0) - MUSIC_END
             for seed in range(200)}
    assert drawn == {1, 2, 3}
    base[0, 1:5] = [5, 4, 3, 2]
    session.write_logits(bf(base))
    drawn = {session.sample(dict(temperature=1.0, top_k=4, top_p=0.01, repetition_penalty=1.0,
                                 min_tokens=0, max_tokens=100), seed, 0) - MUSIC_END
             for seed in range(50)}
    assert drawn == {1}
    session.close()


@pytest.mark.parametrize("phase", ["full", "abc", "semantic"])
@pytest.mark.parametrize("branches,cfg", [(1, 1.0), (2, 1.5)])
def test_sampler_random_configurations(engine_yue2, oracle, phase, branches, cfg):
    # seeded sweep over the sampling space (sampling.cpp:38-134, 247-250):
    # temperature (greedy included), top k on both sides of the split form's
    # 128, top p, repetition penalty and window over a history of the phase's
    # native ids (rows boosted so the penalty matters), min tokens before and
    # after the step, legacy on and off, five logit shapes; every draw
    # identical to the oracle's
    rng = np.random.default_rng(1000 * branches + {"full": 1, "abc": 2, "semantic": 3}[phase])
    session = engine_yue2.session(branches, 64, phase)
    n = session.vocab
    to_native = oracle.lib().oracle_local_to_native
    for trial in range(24):
        sampling = dict(temperature=float(rng.choice([0.0, 0.6, 1.0, 1.4])),
                        top_k=int(rng.choice([1, 7, 50, 100, 130, 400, 3000, 100000])),
                        top_p=float(rng.choice([0.3, 0.8, 0.93, 1.0])),
                        repetition_penalty=float(rng.choice([1.0, 1.1, 1.5])),
                        penalty_window=int(rng.choice([5, 50, 100])),
                        min_tokens=int(rng.choice([0, 10])), max_tokens=9000)
        kind = str(rng.choice(["normal", "ties", "peaked", "flat", "integers"]))
        x = logits_for(rng, kind, branches, n)
        local = rng.integers(0, min(n, 64), size=int(rng.integers(0, 40)))
        hist = [int(to_native(int(t), oracle.PHASES[phase])) for t in local]
        if len(local):  # lift the history's rows to the top so the penalty decides
            import cpu_ref
            f = cpu_ref.bf16_to_f32(x)
            f[:, local] += 4.0
            x = bf(f)
        session.write_logits(x)
        legacy = bool(rng.integers(0, 2))
        seed, step = int(rng.integers(0, 2**62)), int(rng.integers(0, 20))
        got = session.sample(sampling, seed, step, history=hist, cfg_scale=cfg, legacy_off=legacy)
        want = oracle_token(oracle, x, sampling, seed, step, hist, phase, cfg, legacy)
        assert got == want, (trial, sampling, kind, legacy, step, got, want)
    session.close()
