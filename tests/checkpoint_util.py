"""Writers of converted checkpoint directories for the loader tests.

A directory holds conversion.json (the schema-1 manifest of
native/src/conversion.cpp:609-693, reduced to what ARModel reads,
ar.cpp:137-160), config.json and ar-<precision>.safetensors. Tensors are
bf16 bit patterns (uint16) or, for the quantized precisions' codes, uint32. `write_safetensors` writes the format directly
(8-byte little-endian header length, JSON header, data) so that malformed
files can be made; `write_checkpoint(..., writer="safetensors")` uses the
safetensors package instead, to check files made by the official writer.
"""
import json
import os
import struct

import numpy as np


def manifest(precision="bf16"):
    entry = {"ar": f"ar-{precision}.safetensors"}
    if precision == "bf16":
        entry["dtype"] = "bfloat16"
    else:
        entry.update(bits=8 if precision == "8bit" else 4, group_size=64, mode="affine",
                     linear_only=True)
    return {"schema": 1, "format": "lyra-yue2-mlx", "precisions": {precision: entry}}


def hf_config(cfg):
    keys = ("hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
            "num_key_value_heads", "head_dim", "vocab_size", "max_position_embeddings",
            "rms_norm_eps", "rope_theta")
    out = {k: cfg[k] for k in keys}
    out.update(hidden_act="silu", tie_word_embeddings=False, rope_scaling=None,
               model_type="qwen3")
    return out


def _raw(arr):
    """(dtype name, little-endian bytes) of a bf16 (uint16) or U32 (uint32) array."""
    if np.asarray(arr).dtype == np.uint32:
        return "U32", np.ascontiguousarray(arr, dtype="<u4").tobytes()
    return "BF16", np.ascontiguousarray(arr, dtype="<u2").tobytes()


def write_safetensors(path, tensors, dtypes=None, shapes=None, offsets=None, pad_odd=False):
    """tensors: name -> uint16 (BF16) or uint32 (U32) array. dtypes/shapes/offsets
    override header fields; pad_odd puts one byte before the data so that
    tensors sit at odd offsets."""
    dtypes, shapes, offsets = dtypes or {}, shapes or {}, offsets or {}
    header, blobs, pos = {}, [], 1 if pad_odd else 0
    if pad_odd:
        blobs.append(b"\0")
    for name in sorted(tensors):
        kind, raw = _raw(tensors[name])
        header[name] = {"dtype": dtypes.get(name, kind),
                        "shape": list(shapes.get(name, np.shape(tensors[name]))),
                        "data_offsets": list(offsets.get(name, (pos, pos + len(raw))))}
        blobs.append(raw)
        pos += len(raw)
    header["__metadata__"] = {"format": "pt"}
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)


def write_checkpoint(directory, cfg, weights, precision="bf16", writer="raw", manifest_patch=None,
                     config_patch=None, **st_kwargs):
    os.makedirs(directory, exist_ok=True)
    m = manifest(precision)
    if manifest_patch:
        manifest_patch(m)
    with open(os.path.join(directory, "conversion.json"), "w") as f:
        json.dump(m, f)
    c = hf_config(cfg)
    if config_patch:
        config_patch(c)
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(c, f)
    path = os.path.join(directory, f"ar-{precision}.safetensors")
    if writer == "safetensors":
        import torch
        from safetensors.torch import save_file

        def tensor(v):
            if np.asarray(v).dtype == np.uint32:
                return torch.from_numpy(np.ascontiguousarray(v).view(np.int32)).view(torch.uint32)
            return torch.from_numpy(np.ascontiguousarray(v, dtype=np.uint16).view(np.int16)).view(
                torch.bfloat16)

        save_file({k: tensor(v) for k, v in weights.items()}, path)
    else:
        write_safetensors(path, weights, **st_kwargs)
    return directory
