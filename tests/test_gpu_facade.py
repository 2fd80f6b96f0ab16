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
    assert cases["cancelled"]["error"] == "InterruptedError" and cases["cancelled"]["calls"] == 3
    assert cases["throwing"]["error"] == "out_of_range" and cases["throwing"]["what"] == "boom"
    assert cases["again"]["tokens"] == greedy
