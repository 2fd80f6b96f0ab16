"""The compiled C++ facade (include/yuear.hpp) on the GPU.

tests/cxx/facade_test.cpp (built by the package Makefile into
yue2-mlx_amd/yuear_facade_test) calls generate_tokens with the reference's
C++ signature (ar.hpp:43-48) the way Pipeline::generate_phase does
(pipeline.cpp:186-211): greedy, sampled with a per-token callback, CFG with a
negative prefix, invalid sampling, cancellation from the `cancelled` poll and
an exception thrown by the callback. Its tokens must equal the Python
binding's on the same engine (deterministic generator, seed 11), its errors
carry the reference's types (ValueError; InterruptedError for a cancelled
run, sampling.cpp:243), a callback's exception reaches the caller, and the
engine generates again afterwards.
"""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "yue2-mlx_amd", "yuear_facade_test")
CFG = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, head_dim=128, vocab_size=512, max_position_embeddings=64,
           rms_norm_eps=1e-5, rope_theta=500000.0)
PREFIX = [3, 17, 255, 1, 98]
GREEDY = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0, penalty_window=50,
              min_tokens=0, max_tokens=24)
SAMPLED = dict(temperature=1.0, top_p=0.9, top_k=40, repetition_penalty=1.1, penalty_window=50,
               min_tokens=0, max_tokens=24)


def test_cxx_facade_matches_python_binding(yuear_lib):
    assert os.path.exists(BINARY), "build the package first (make -C yue2-mlx_amd)"
    print("[facade] running", BINARY, flush=True)
    run = subprocess.run([BINARY], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    cases = {c["case"]: c for c in map(json.loads, run.stdout.strip().splitlines())}
    engine = yuear_lib.Engine(CFG, yuear_lib.random_weights(CFG, 11, std=0.02, norm_std=0.1))
    greedy, _, _ = engine.generate_tokens(PREFIX, GREEDY, 0)
    sampled, _, _ = engine.generate_tokens(PREFIX, SAMPLED, 77)
    cfg, _, _ = engine.generate_tokens(PREFIX, SAMPLED, 78, negative=[9, 8, 7], cfg_scale=1.5)
    engine.close()
    assert cases["greedy"]["tokens"] == greedy and len(greedy) == 24
    assert cases["greedy"]["truncated"] is True  # "full" has no end token
    timing = cases["greedy"]["timing"]
    for key in ("output_tokens", "output_tps", "execution"):
        assert key in timing
    assert cases["sampled"]["tokens"] == sampled
    assert cases["sampled"]["callback"] == sampled and cases["sampled"]["phase"] == "full"
    assert cases["cfg"]["tokens"] == cfg
    assert cases["invalid"]["error"] == "ValueError"
    # the reference's cancellation points and messages (sampling.cpp:156,
    # 164, 206, 243): nothing is reported once a poll has seen the cancel
    expect = {"cancel_before": ("Cancelled before prefill", 0, 1),
              "cancel_branch1": ("Cancelled before prefill", 0, 4),
              "cancel_prefill": ("Cancelled during prefill", 0, 5),
              "cancelled": ("Cancelled during full", 3, None)}
    for name, (message, calls, polls) in expect.items():
        case = cases[name]
        assert case["error"] == "InterruptedError", case
        assert case["message"] == message and case["calls"] == calls, case
        if polls is not None:
            assert case["polls"] == polls, case
    assert cases["throwing"]["error"] == "out_of_range" and cases["throwing"]["what"] == "boom"
    assert cases["again"]["tokens"] == greedy


PIPELINE = os.path.join(ROOT, "yue2-mlx_amd", "yuear_pipeline_test")
YUE2_TINY = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                 num_attention_heads=4, num_key_value_heads=2, head_dim=128, vocab_size=184704,
                 max_position_embeddings=1024, rms_norm_eps=1e-5, rope_theta=500000.0)
ABC = dict(temperature=0.7, top_p=0.9, top_k=30, repetition_penalty=1.005, penalty_window=100,
           min_tokens=4, max_tokens=16)
SEMANTIC = dict(temperature=1.0, top_p=0.95, top_k=100, repetition_penalty=1.2,
                penalty_window=50, min_tokens=4, max_tokens=12)


def test_cxx_pipeline_glue(yuear_lib, text_vocab):
    """yuear::Pipeline (pipeline.cpp:186-263) composed from the parts the
    other tests hold to the oracle: its prefixes are token_prefixes of the
    request and of the ABC ids the abc phase produced (whose text is their
    decode), the semantic phase runs with the negative prefix when the
    guidance is not 1 and with the legacy-off sampler for cot "off", and
    its codec frames are the semantic tokens less CODEC_OFFSET."""
    import text_ref
    assert os.path.exists(PIPELINE), "build the package first (make -C yue2-mlx_amd)"
    path, ranks = text_vocab
    print("[facade] running", PIPELINE, flush=True)
    run = subprocess.run([PIPELINE, path], capture_output=True, text=True, timeout=180)
    assert run.returncode == 0, run.stderr
    cases = {c["case"]: c for c in map(json.loads, run.stdout.strip().splitlines())}
    tok = yuear_lib.Tokenizer(path)
    engine = yuear_lib.Engine(YUE2_TINY, seed=13, std=0.02, norm_std=0.1)
    style, lyrics = "female vocal, pop, piano", "[verse]\nI've been walking down this road tonight\n"

    # generated score, guidance 1.5
    full = yuear_lib.SongRequest(style, lyrics, seed=21, cfg_scale=1.5)
    start = yuear_lib.token_prefixes(full, tok)
    assert start == text_ref.token_prefixes(style, lyrics, "full", ranks)
    abc_ids, _, truncated = engine.generate_tokens(start, ABC, 21, phase="abc")
    plan = cases["plan_full"]
    assert plan["abc_ids"] == abc_ids and all(0 <= t < text_ref.EOD for t in abc_ids)
    assert plan["abc"] == tok.decode(abc_ids) == text_ref.decode(abc_ids, ranks)
    assert plan["prefix"] == yuear_lib.token_prefixes(full, tok, abc_ids)
    assert plan["truncated"] == truncated and plan["timing"]["output_tokens"] == len(abc_ids)
    negative = yuear_lib.negative_prefix(full, tok, abc_ids)
    codes, _, _ = engine.generate_tokens(plan["prefix"], SEMANTIC, 21, phase="semantic",
                                         negative=negative, cfg_scale=1.5)
    assert cases["semantic_full"]["codes"] == [t - 151853 for t in codes]
    assert all(0 <= c < 32768 for c in cases["semantic_full"]["codes"])

    # cot off: no abc phase, guidance 1.01, legacy-off sampling
    off = yuear_lib.SongRequest(style, lyrics, cot="off", seed=21)
    assert cases["plan_off"]["prefix"] == yuear_lib.token_prefixes(off, tok)
    assert cases["plan_off"]["abc_ids"] == [] and cases["plan_off"]["abc"] is None
    codes, _, _ = engine.generate_tokens(cases["plan_off"]["prefix"], SEMANTIC, 21,
                                         phase="semantic", negative=yuear_lib.negative_prefix(off, tok),
                                         cfg_scale=1.01, legacy_off=True)
    assert cases["semantic_off"]["codes"] == [t - 151853 for t in codes]

    # the request's own score
    abc = "X:1\nK:C\n\"C\"CDEF|GABc|\n"
    given = yuear_lib.SongRequest(style, lyrics, cot="melody", seed=21, abc=abc)
    ext = cases["plan_external"]
    assert ext["abc_ids"] == tok.encode(abc) == text_ref.encode(abc, ranks)
    assert ext["abc"] == abc and ext["prefix"] == yuear_lib.token_prefixes(given, tok)
    assert ext["timing"] == {"seconds": 0.0, "output_tokens": 0,
                             "external_prefix_tokens": len(ext["abc_ids"])}
    codes, _, _ = engine.generate_tokens(ext["prefix"], SEMANTIC, 21, phase="semantic")
    assert cases["semantic_external"]["codes"] == [t - 151853 for t in codes]

    assert cases["tampered"]["error"] == "ValueError"
    assert cases["tampered"]["message"] == "Plan prefix disagrees with request/exact ABC IDs"
    assert cases["invalid_request"]["error"] == "ValueError"
    assert cases["invalid_request"]["message"] == "id must be a filename-safe identifier"
    assert cases["budget"]["error"] == "ValueError"
    assert "exceeds 24576" in cases["budget"]["message"]
    engine.close()
    tok.close()
