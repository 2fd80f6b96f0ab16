"""Checkpoint directory loader on the GPU: an engine loaded from
conversion.json + config.json + ar-bf16.safetensors (ar.cpp:133-238) decodes
bit for bit like the engine built from the same host tensors, for files from
the safetensors package and from a raw writer with tensors at odd offsets."""
import numpy as np
import pytest

from checkpoint_util import write_checkpoint
from conftest import TINY

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("writer,pad_odd", [("safetensors", False), ("raw", True)])
def test_loaded_engine_matches_host_tensors(yuear_lib, tmp_path, writer, pad_odd):
    print(f"[checkpoint] writer={writer} pad_odd={pad_odd}", flush=True)
    weights = yuear_lib.random_weights(TINY, seed=12, norm_std=0.1)
    kw = {"pad_odd": True} if pad_odd else {}
    d = write_checkpoint(tmp_path / "ck", TINY, weights, writer=writer, **kw)
    loaded = yuear_lib.Engine.load(str(d))
    direct = yuear_lib.Engine(TINY, weights)
    try:
        assert loaded.config["hidden_size"] == TINY["hidden_size"]
        prompt, steps = [5, 77, 301, 12, 9], [44, 500, 3]
        out = []
        for e in (loaded, direct):
            s = e.session(1, 32)
            out.append([s.prefill(0, prompt)] + [s.step(t)[0] for t in steps])
            s.close()
        for a, b in zip(*out):
            np.testing.assert_array_equal(a, b)
    finally:
        loaded.close()
        direct.close()
