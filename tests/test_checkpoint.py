"""Checkpoint directory loader (ARModel(directory, precision), ar.cpp:133-238)
on the CPU, for the bf16 and the affine-quantized ("8bit" / "4bit")
precisions: yuear_checkpoint_inspect reads and validates conversion.json,
config.json and the safetensors header without touching the GPU. Every
message checked here is the reference's own (ar.cpp:137-236)."""
import json
import os

import numpy as np
import pytest

from checkpoint_util import write_checkpoint, write_safetensors
from conftest import TINY
from quant_util import quantize_model


@pytest.fixture(scope="module")
def weights(yuear_lib):
    return yuear_lib.random_weights(TINY, seed=4, norm_std=0.1)


def inspect(yuear_lib, d, precision="bf16", strict=False):
    return yuear_lib.inspect_checkpoint(str(d), precision, strict)


@pytest.mark.parametrize("writer", ["raw", "safetensors"])
def test_inspect_returns_the_architecture(yuear_lib, weights, tmp_path, writer):
    d = write_checkpoint(tmp_path / "ck", TINY, weights, writer=writer)
    cfg = inspect(yuear_lib, d)
    for k in ("hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
              "num_key_value_heads", "head_dim", "vocab_size", "max_position_embeddings"):
        assert cfg[k] == TINY[k], k
    assert cfg["rms_norm_eps"] == pytest.approx(TINY["rms_norm_eps"])
    assert cfg["rope_theta"] == TINY["rope_theta"] and cfg["qk_norm"]


def test_max_position_embeddings_defaults_to_the_context(yuear_lib, weights, tmp_path):
    d = write_checkpoint(tmp_path, TINY, weights,
                         config_patch=lambda c: c.pop("max_position_embeddings"))
    assert inspect(yuear_lib, d)["max_position_embeddings"] == 24576


def test_strict_requires_the_yue2_dimensions(yuear_lib, weights, tmp_path):
    d = write_checkpoint(tmp_path, TINY, weights)
    with pytest.raises(ValueError, match="Incompatible YuE2 config: hidden_size"):
        inspect(yuear_lib, d, strict=True)


def test_strict_accepts_the_yue2_config_and_checks_integers(yuear_lib, tmp_path):
    # config and manifest only (the 6 GB tensor file is not needed to see the
    # config checks pass: the loader then stops at the missing file)
    yue2 = dict(hidden_size=2048, intermediate_size=6144, num_hidden_layers=28,
                num_attention_heads=16, num_key_value_heads=8, head_dim=128, vocab_size=184704,
                max_position_embeddings=24576, rms_norm_eps=1e-6, rope_theta=1e6)
    d = tmp_path / "yue2"
    write_checkpoint(d, yue2, {})
    os.remove(d / "ar-bf16.safetensors")
    with pytest.raises(FileNotFoundError, match="ar-bf16.safetensors"):
        inspect(yuear_lib, d, strict=True)
    cfg = json.loads((d / "config.json").read_text())
    cfg["hidden_size"] = 2048.0
    (d / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="Generator config field hidden_size must be a positive"):
        inspect(yuear_lib, d, strict=True)


@pytest.mark.parametrize("patch,kind,message", [
    (lambda c: c.update(tie_word_embeddings=True), ValueError, "untied input and output"),
    (lambda c: c.update(rope_scaling={"type": "linear", "factor": 2.0}), ValueError,
     "fixed base RoPE without scaling"),
    (lambda c: c.update(hidden_act="gelu"), ValueError, "hidden_act must be silu"),
    (lambda c: c.update(rms_norm_eps=0), ValueError, "rms_norm_eps must be finite and positive"),
    (lambda c: c.pop("rms_norm_eps"), ValueError, "rms_norm_eps must be finite and positive"),
    (lambda c: c.update(num_hidden_layers=-2), ValueError,
     "num_hidden_layers must be a positive integer"),
    (lambda c: c.update(rope_theta="big"), ValueError, "rope_theta"),
])
def test_config_checks(yuear_lib, weights, tmp_path, patch, kind, message):
    d = write_checkpoint(tmp_path, TINY, weights, config_patch=patch)
    with pytest.raises(kind, match=message):
        inspect(yuear_lib, d)


def test_rope_scaling_null_or_empty_is_accepted(yuear_lib, weights, tmp_path):
    for i, v in enumerate((None, {})):
        d = write_checkpoint(tmp_path / str(i), TINY, weights,
                             config_patch=lambda c, v=v: c.update(rope_scaling=v))
        inspect(yuear_lib, d)


@pytest.mark.parametrize("patch,kind,message", [
    (lambda m: m.update(schema=2), ValueError, "schema-1 manifest"),
    (lambda m: m["precisions"]["bf16"].update(ar="ar.safetensors"), ValueError,
     "Manifest AR filename does not match precision"),
    (lambda m: m["precisions"]["bf16"].update(dtype="float16"), ValueError,
     "must declare dtype='bfloat16'"),
    (lambda m: m["precisions"].clear(), FileNotFoundError,
     "does not contain bf16 AR weights"),
])
def test_manifest_checks(yuear_lib, weights, tmp_path, patch, kind, message):
    d = write_checkpoint(tmp_path, TINY, weights, manifest_patch=patch)
    with pytest.raises(kind, match=message):
        inspect(yuear_lib, d)


@pytest.mark.parametrize("writer", ["raw", "safetensors"])
@pytest.mark.parametrize("precision,bits", [("8bit", 8), ("4bit", 4)])
def test_quantized_precisions_are_accepted(yuear_lib, weights, tmp_path, writer, precision, bits):
    q = quantize_model(weights, bits)
    d = write_checkpoint(tmp_path / "q", TINY, q, precision=precision, writer=writer)
    assert inspect(yuear_lib, d, precision)["hidden_size"] == TINY["hidden_size"]
    # the bf16 file of the same directory is not what the manifest names
    with pytest.raises(FileNotFoundError, match="does not contain bf16 AR weights"):
        inspect(yuear_lib, d, "bf16")


@pytest.mark.parametrize("bits", [8, 4])
def test_quantized_tensor_checks(yuear_lib, weights, tmp_path, bits):
    precision = f"{bits}bit"
    q = quantize_model(weights, bits)
    name = "model.layers.0.mlp.down_proj"
    H, F = TINY["hidden_size"], TINY["intermediate_size"]
    cases = [
        # bf16 codes where U32 is required (an unquantized linear in a quantized file)
        (dict(q, **{name + ".weight": weights[name + ".weight"]}),
         {}, f"Incompatible AR tensor shape/dtype: {name}.weight"),
        (q, {"shapes": {name + ".weight": (H, F * bits // 32 + 1)}},
         f"Incompatible AR tensor shape/dtype: {name}.weight"),
        (q, {"dtypes": {name + ".scales": "F16"}}, f"Incompatible AR tensor shape/dtype: {name}.scales"),
        ({k: v for k, v in q.items() if k != name + ".biases"}, {}, f"Missing AR tensor: {name}.biases"),
        (dict(q, **{"model.norm.scales": np.zeros(4, np.uint16)}), {},
         "Unexpected AR tensor: model.norm.scales"),
        (q, {"offsets": {name + ".weight": (0, 4)}}, f"invalid data offsets for {name}.weight"),
    ]
    for i, (tensors, kw, message) in enumerate(cases):
        d = write_checkpoint(tmp_path / str(i), TINY, {}, precision=precision)
        write_safetensors(d / f"ar-{precision}.safetensors", tensors, **kw)
        with pytest.raises(ValueError, match=message):
            inspect(yuear_lib, d, precision)


def test_quantized_settings_and_precision_names(yuear_lib, weights, tmp_path):
    d = write_checkpoint(tmp_path / "g", TINY, weights, precision="8bit",
                         manifest_patch=lambda m: m["precisions"]["8bit"].update(group_size=32))
    with pytest.raises(ValueError, match="Invalid affine quantization settings"):
        inspect(yuear_lib, d, "8bit")
    with pytest.raises(ValueError, match="precision must be"):
        inspect(yuear_lib, d, "fp8")


def test_missing_files(yuear_lib, weights, tmp_path):
    with pytest.raises(FileNotFoundError):
        inspect(yuear_lib, tmp_path / "nowhere")
    d = write_checkpoint(tmp_path / "c", TINY, weights)
    os.remove(d / "config.json")
    with pytest.raises(FileNotFoundError, match="config.json"):
        inspect(yuear_lib, d)


def test_tensor_checks(yuear_lib, weights, tmp_path):
    name = "model.layers.1.mlp.up_proj.weight"
    cases = []
    missing = dict(weights)
    missing.pop(name)
    cases.append((dict(tensors=missing), f"Missing AR tensor: {name}"))
    extra = dict(weights, **{"model.layers.1.mlp.bias": np.zeros(4, np.uint16)})
    cases.append((dict(tensors=extra), "Unexpected AR tensor: model.layers.1.mlp.bias"))
    cases.append((dict(tensors=weights, dtypes={name: "F16"}),
                  f"Incompatible AR tensor shape/dtype: {name}"))
    cases.append((dict(tensors=weights, shapes={name: (512, 255)}),
                  f"Incompatible AR tensor shape/dtype: {name}"))
    cases.append((dict(tensors=weights, offsets={name: (0, 10)}),
                  f"invalid data offsets for {name}"))
    cases.append((dict(tensors=weights, offsets={name: (10 ** 12, 10 ** 12 + 512 * 256 * 2)}),
                  f"invalid data offsets for {name}"))
    for i, (kw, message) in enumerate(cases):
        d = write_checkpoint(tmp_path / str(i), TINY, {})
        write_safetensors(d / "ar-bf16.safetensors", **kw)
        with pytest.raises(ValueError, match=message):
            inspect(yuear_lib, d)


def test_malformed_header(yuear_lib, weights, tmp_path):
    d = write_checkpoint(tmp_path, TINY, weights)
    path = d / "ar-bf16.safetensors"
    data = path.read_bytes()
    path.write_bytes(data[:5])
    with pytest.raises(ValueError, match="truncated safetensors header"):
        inspect(yuear_lib, d)
    path.write_bytes((10 ** 9).to_bytes(8, "little") + data[8:])
    with pytest.raises(ValueError, match="invalid safetensors header length"):
        inspect(yuear_lib, d)
    path.write_bytes((5).to_bytes(8, "little") + b"{oops" + data[13:])
    with pytest.raises(ValueError, match="invalid JSON"):
        inspect(yuear_lib, d)
