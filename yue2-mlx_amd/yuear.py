"""Python binding of libyuear (the gfx950 AR decode library) over its C ABI.

Mirrors the reference's decode interfaces so callers and tests read alike:
``Engine.generate_tokens`` follows ``generate_tokens`` (native/src/sampling.cpp
:185-288; oracle/port/lyra/ar.py:614-729) and ``Session`` follows the GraphAR
decode-step object (vendor/yue/src/yue2/cuda_graph.py:35-240): ``prefill`` per
branch, then ``step(token)`` returning logits, then ``close``.

Errors map to the reference's exception types: status 2 -> ValueError,
130 -> InterruptedError, 1 -> RuntimeError. There is no CPU fallback: when the
library is missing this module raises at import.
"""
from __future__ import annotations

import ctypes as C
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libyuear.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "yuear.h")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C yue2-mlx_amd)")

u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
i32p = C.POINTER(C.c_int32)
DTYPE_BF16, DTYPE_U32 = 0, 1  # YUEAR_DTYPE_*


class ModelConfig(C.Structure):
    _fields_ = [("hidden_size", C.c_int32), ("intermediate_size", C.c_int32),
                ("num_hidden_layers", C.c_int32), ("num_attention_heads", C.c_int32),
                ("num_key_value_heads", C.c_int32), ("head_dim", C.c_int32),
                ("vocab_size", C.c_int32), ("max_position_embeddings", C.c_int32),
                ("rms_norm_eps", C.c_float), ("rope_theta", C.c_double), ("qk_norm", C.c_int32)]


class SamplingC(C.Structure):
    _fields_ = [("temperature", C.c_double), ("top_p", C.c_double), ("top_k", C.c_int32),
                ("repetition_penalty", C.c_double), ("penalty_window", C.c_int32),
                ("min_tokens", C.c_int32), ("max_tokens", C.c_int32)]


class TensorC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.c_void_p), ("numel", C.c_int64),
                ("dtype", C.c_int32)]


class WeightSource(C.Structure):
    _fields_ = [("kind", C.c_int32), ("seed", C.c_uint64), ("std", C.c_float),
                ("norm_std", C.c_float), ("tensors", C.POINTER(TensorC)), ("count", C.c_int32),
                ("bits", C.c_int32)]


class SongRequestC(C.Structure):
    _fields_ = [("style", C.c_char_p), ("lyrics", C.c_char_p), ("cot", C.c_char_p),
                ("abc", C.c_char_p), ("id", C.c_char_p), ("seed", C.c_uint64),
                ("cfg_scale", C.c_double), ("has_cfg_scale", C.c_int32)]


TOKEN_CB = C.CFUNCTYPE(None, C.c_void_p, C.c_char_p, C.c_int32)
CANCEL_POLL = C.CFUNCTYPE(C.c_int32, C.c_void_p)

lib = C.CDLL(LIB_PATH)
_P = C.POINTER
_SIGS = {
    "yuear_build_identifier": (C.c_char_p, []),
    "yuear_string_free": (None, [C.c_void_p]),
    "yuear_engine_create": (C.c_int, [_P(ModelConfig), _P(WeightSource), _P(C.c_void_p),
                                      _P(C.c_void_p)]),
    "yuear_engine_destroy": (None, [C.c_void_p]),
    "yuear_checkpoint_inspect": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int32, _P(ModelConfig),
                                           _P(C.c_void_p)]),
    "yuear_engine_load": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int32, _P(C.c_void_p),
                                    _P(C.c_void_p)]),
    "yuear_engine_cancel": (None, [C.c_void_p]),
    "yuear_engine_bits": (C.c_int32, [C.c_void_p]),
    "yuear_quantize_affine": (None, [u16p, C.c_int64, C.c_int32, C.c_int32, u32p, u16p, u16p]),
    "yuear_tensor_id": (C.c_int32, [C.c_char_p]),
    "yuear_random_tensor": (None, [C.c_uint64, C.c_int32, C.c_float, C.c_float, C.c_int64,
                                   u16p]),
    "yuear_rope_table": (None, [C.c_int32, C.c_int32, C.c_double, u16p, u16p]),
    "yuear_generate_tokens": (C.c_int, [C.c_void_p, i32p, C.c_int32, _P(SamplingC), C.c_uint64,
                                        C.c_char_p, i32p, C.c_int32, C.c_double, C.c_int32,
                                        CANCEL_POLL, TOKEN_CB, C.c_void_p, i32p, i32p, i32p,
                                        _P(C.c_void_p),
                                        _P(C.c_void_p)]),
    "yuear_session_begin": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_char_p,
                                      _P(C.c_void_p), _P(C.c_void_p)]),
    "yuear_session_end": (None, [C.c_void_p]),
    "yuear_session_prefill": (C.c_int, [C.c_void_p, C.c_int32, i32p, C.c_int32, u16p,
                                        _P(C.c_void_p)]),
    "yuear_session_step": (C.c_int, [C.c_void_p, i32p, u16p, _P(C.c_void_p)]),
    "yuear_session_sample": (C.c_int, [C.c_void_p, _P(SamplingC), C.c_uint64, C.c_double,
                                       C.c_int32, C.c_int32, i32p, C.c_int32, i32p,
                                       _P(C.c_void_p)]),
    "yuear_session_position": (C.c_int32, [C.c_void_p, C.c_int32]),
    "yuear_session_phase_size": (C.c_int32, [C.c_void_p]),
    "yuear_session_write_kv": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, u16p, u16p,
                                         C.c_int32, _P(C.c_void_p)]),
    "yuear_session_read_kv": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, u16p, u16p,
                                        C.c_int32, _P(C.c_void_p)]),
    "yuear_session_write_logits": (C.c_int, [C.c_void_p, u16p, _P(C.c_void_p)]),
    "yuear_session_set_position": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, _P(C.c_void_p)]),
    "yuear_session_layer_step": (C.c_int, [C.c_void_p, C.c_int32, u16p, u16p, _P(C.c_void_p)]),
    "yuear_session_time_steps": (C.c_int, [C.c_void_p, C.c_int32, _P(C.c_double),
                                           _P(C.c_void_p)]),
    "yuear_session_time_generate": (C.c_int, [C.c_void_p, _P(SamplingC), C.c_uint64, C.c_int32,
                                              C.c_int32, _P(C.c_double), i32p, _P(C.c_void_p)]),
    "yuear_session_time_kernel": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int32, _P(C.c_double),
                                            _P(C.c_void_p)]),
    "yuear_op_gemv": (C.c_int32, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                                  C.c_int32, C.c_void_p, C.c_float, C.c_void_p, C.c_int32,
                                  C.c_int32, C.c_void_p]),
    "yuear_op_attention_decode": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_float,
                                              C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                              C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                              C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]),
    "yuear_op_attention_decode_noalloc": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_void_p,
                                                      C.c_float, C.c_void_p, C.c_void_p,
                                                      C.c_void_p, C.c_void_p, C.c_void_p,
                                                      C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                                      C.c_int32, C.c_void_p, C.c_void_p]),
    "yuear_op_qgemv": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                   C.c_int32, C.c_void_p, C.c_int32, C.c_void_p, C.c_float,
                                   C.c_void_p, C.c_int32, C.c_int32, C.c_void_p]),
    "yuear_op_dequantize": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                        C.c_int32, C.c_void_p, C.c_void_p]),
    "yuear_nar_attention_workspace_bytes": (C.c_int64, [C.c_int32, C.c_int32, C.c_int32]),
    "yuear_nar_condition": (C.c_int, [C.c_void_p, i32p, C.c_int32, C.c_int32, C.c_void_p,
                                      C.c_void_p, i32p, _P(C.c_void_p)]),
    "yuear_nar_attention": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                      C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                      C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                      _P(C.c_void_p)]),
    "yuear_op_gemm": (C.c_int32, [C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int32,
                                  C.c_int32, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p]),
    "yuear_op_gemm_tile": (C.c_int32, [C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int32,
                                       C.c_int32, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                       C.c_void_p]),
    "yuear_op_gemm_split": (C.c_int32, [C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int32,
                                        C.c_int32, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                        C.c_int32, C.c_void_p]),
    "yuear_op_attention_prefill": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                                               C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                               C.c_void_p, C.c_void_p]),
    "yuear_tokenizer_load": (C.c_int, [C.c_char_p, _P(C.c_void_p), _P(C.c_void_p)]),
    "yuear_tokenizer_destroy": (None, [C.c_void_p]),
    "yuear_tokenizer_encode": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int64, _P(i32p),
                                         _P(C.c_int64), _P(C.c_void_p)]),
    "yuear_tokenizer_decode": (C.c_int, [C.c_void_p, i32p, C.c_int64, _P(C.c_void_p),
                                         _P(C.c_int64), _P(C.c_void_p)]),
    "yuear_ids_free": (None, [i32p]),
    "yuear_text_nfc": (C.c_int, [C.c_char_p, C.c_int64, _P(C.c_void_p), _P(C.c_int64),
                                 _P(C.c_void_p)]),
    "yuear_text_pieces": (C.c_int, [C.c_char_p, C.c_int64, _P(i32p), _P(C.c_int64),
                                    _P(C.c_void_p)]),
    "yuear_song_request_validate": (C.c_int, [_P(SongRequestC), _P(C.c_void_p)]),
    "yuear_song_request_guidance": (C.c_double, [_P(SongRequestC)]),
    "yuear_token_prefixes": (C.c_int, [C.c_void_p, _P(SongRequestC), i32p, C.c_int64, C.c_int32,
                                       _P(i32p), _P(C.c_int64), _P(C.c_void_p)]),
    "yuear_negative_prefix": (C.c_int, [C.c_void_p, _P(SongRequestC), i32p, C.c_int64,
                                        C.c_int32, _P(i32p), _P(C.c_int64), _P(C.c_void_p)]),
    "yuear_chunk_ranges": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, _P(i32p), _P(C.c_int64),
                                     _P(C.c_void_p)]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype, _fn.argtypes = _res, _args

EXPORTS = tuple(_SIGS)


def _take_error(err):
    if not err.value:
        return {"type": "RuntimeError", "message": "unknown error"}
    text = C.cast(err, C.c_char_p).value.decode()
    lib.yuear_string_free(err)
    try:
        return json.loads(text)
    except ValueError:
        return {"type": "RuntimeError", "message": text}


class TextDecodeError(ValueError):
    """The library's UnicodeDecodeError (invalid UTF-8 input text)."""


def _check(status, err):
    if status == 0:
        return
    info = _take_error(err)
    kind = {"ValueError": ValueError, "InterruptedError": InterruptedError,
            "FileNotFoundError": FileNotFoundError, "PermissionError": PermissionError,
            "OSError": OSError, "UnicodeDecodeError": TextDecodeError,
            "MemoryError": MemoryError}.get(info.get("type"), RuntimeError)
    if status == 130:
        kind = InterruptedError
    raise kind(info.get("message", ""))


def build_identifier():
    return lib.yuear_build_identifier().decode()


# ---- configs and weights ----

LAYER_SUFFIXES = ("input_layernorm", "post_attention_layernorm", "self_attn.q_norm",
                  "self_attn.k_norm", "self_attn.q_proj", "self_attn.k_proj",
                  "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj",
                  "mlp.down_proj")


def tensor_shapes(config: dict) -> dict:
    """Reference tensor names and shapes (native/src/ar.cpp:216-233)."""
    H, F, V = config["hidden_size"], config["intermediate_size"], config["vocab_size"]
    Hq, Hkv, D = config["num_attention_heads"], config["num_key_value_heads"], config["head_dim"]
    shapes = {"model.embed_tokens.weight": (V, H), "model.norm.weight": (H,),
              "lm_head.weight": (V, H)}
    per = {"input_layernorm": (H,), "post_attention_layernorm": (H,), "self_attn.q_norm": (D,),
           "self_attn.k_norm": (D,), "self_attn.q_proj": (Hq * D, H),
           "self_attn.k_proj": (Hkv * D, H), "self_attn.v_proj": (Hkv * D, H),
           "self_attn.o_proj": (H, Hq * D), "mlp.gate_proj": (F, H), "mlp.up_proj": (F, H),
           "mlp.down_proj": (H, F)}
    for i in range(config["num_hidden_layers"]):
        for suffix in LAYER_SUFFIXES:
            shapes[f"model.layers.{i}.{suffix}.weight"] = per[suffix]
    return shapes


def random_tensor(name, shape, seed, std=0.02, norm_std=0.0):
    """The generator's bytes for one tensor: N(0, std) weights, 1 + N(0,
    norm_std) norm gains (bf16 bit patterns)."""
    tid = lib.yuear_tensor_id(name.encode())
    if tid < 0:
        raise ValueError(f"unknown tensor {name}")
    out = np.empty(shape, dtype=np.uint16)
    gain = "norm" in name
    lib.yuear_random_tensor(seed, tid, 1.0 if gain else 0.0, norm_std if gain else std,
                            out.size, out.ctypes.data_as(u16p))
    return out


def random_normal(seed, tensor_id, shape, mean=0.0, std=1.0):
    """Generator bytes for an arbitrary stream id (inputs such as KV caches)."""
    out = np.empty(shape, dtype=np.uint16)
    lib.yuear_random_tensor(seed, tensor_id, mean, std, out.size, out.ctypes.data_as(u16p))
    return out


def nar_attention(q, k, v, causal=False, query_chunk_size=64, workspace=None, stream=None):
    """nar_attention(query, key, value, causal, query_chunk_size)
    (nar_attention.cpp:224-270) on device tensors: q [B, Hq, Lq, 128], k / v
    [B, Hkv, Lk, 128], torch bf16 on the GPU (plumbing only; the work is
    libyuear's kernel). Returns the output tensor (q's shape)."""
    import torch
    B, Hq, Lq, Dh = q.shape
    _, Hkv, Lk, _ = k.shape
    out = torch.empty_like(q)
    if workspace is None:
        nbytes = lib.yuear_nar_attention_workspace_bytes(B, Hkv, Lk)
        workspace = torch.empty(max(nbytes, 2) // 2, dtype=torch.bfloat16, device=q.device)
    err = C.c_void_p()
    _check(lib.yuear_nar_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), B, Hq, Hkv, Lq, Lk,
                                   Dh, int(causal), int(query_chunk_size), workspace.data_ptr(),
                                   out.data_ptr(), stream, C.byref(err)), err)
    return out


def quantize_affine(w, bits):
    """bf16 rows [rows][k] -> (uint32 codes [rows][k * bits / 32], bf16 scales
    and biases [rows][k / 64]) as the engine's RANDOM source quantizes them
    (mx::quantize(w, 64, bits, "affine"), conversion.cpp:508)."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    rows, k = w.shape
    codes = np.empty((rows, k * bits // 32), dtype=np.uint32)
    scales = np.empty((rows, k // 64), dtype=np.uint16)
    biases = np.empty_like(scales)
    lib.yuear_quantize_affine(w.ctypes.data_as(u16p), rows, k, bits, codes.ctypes.data_as(u32p),
                              scales.ctypes.data_as(u16p), biases.ctypes.data_as(u16p))
    return codes, scales, biases


def quantized_weights(weights, bits):
    """The weight dict of the "8bit" / "4bit" precision made from a bf16 one:
    every projection and the lm_head through `quantize_affine` (ar.cpp:209-214),
    the embedding and the norms unchanged."""
    out = {}
    for name, value in weights.items():
        base = name[:-len(".weight")]
        if base == "lm_head" or base.endswith("_proj"):
            out[name], out[base + ".scales"], out[base + ".biases"] = quantize_affine(value, bits)
        else:
            out[name] = value
    return out


def random_weights(config, seed, std=0.02, norm_std=0.0):
    return {name: random_tensor(name, shape, seed, std, norm_std)
            for name, shape in tensor_shapes(config).items()}


V_BLOCK = 32  # slots per block of the V cache layout


def kv_slots(capacity):
    """Slots per kv head of a cache of `capacity` positions (whole V blocks)."""
    return (capacity + V_BLOCK - 1) // V_BLOCK * V_BLOCK


def v_blocked(v):
    """[..., slots, 128] values (slots a multiple of 32) -> the V cache layout
    of the op-level attention entry points: 32-slot blocks stored dim-major,
    element (t, d) at (t // 32) * 4096 + d * 32 + t % 32 (same shape)."""
    v = np.asarray(v)
    *lead, n, d = v.shape
    if n % V_BLOCK:
        raise ValueError("slots must be a multiple of 32")
    return np.ascontiguousarray(
        v.reshape(*lead, n // V_BLOCK, V_BLOCK, d).swapaxes(-1, -2)).reshape(*lead, n, d)


def v_unblocked(vb):
    """Inverse of v_blocked."""
    vb = np.asarray(vb)
    *lead, n, d = vb.shape
    return np.ascontiguousarray(
        vb.reshape(*lead, n // V_BLOCK, d, V_BLOCK).swapaxes(-1, -2)).reshape(*lead, n, d)


def rope_table(positions, head_dim, theta):
    c = np.empty((positions, head_dim // 2), dtype=np.uint16)
    s = np.empty_like(c)
    lib.yuear_rope_table(positions, head_dim, theta, c.ctypes.data_as(u16p),
                         s.ctypes.data_as(u16p))
    return c, s


def _config_struct(config):
    return ModelConfig(config["hidden_size"], config["intermediate_size"],
                       config["num_hidden_layers"], config["num_attention_heads"],
                       config["num_key_value_heads"], config["head_dim"], config["vocab_size"],
                       config.get("max_position_embeddings", 24576), config["rms_norm_eps"],
                       config["rope_theta"], int(config.get("qk_norm", True)))


def sampling_struct(sampling):
    s = dict(temperature=1.0, top_p=0.95, top_k=100, repetition_penalty=1.2, penalty_window=50,
             min_tokens=200, max_tokens=9000)  # types.hpp:29-33 defaults
    if sampling is not None:
        s.update(sampling if isinstance(sampling, dict) else vars(sampling))
    return SamplingC(s["temperature"], s["top_p"], s["top_k"], s["repetition_penalty"],
                     s["penalty_window"], s["min_tokens"], s["max_tokens"])


def _i32(seq):
    arr = np.ascontiguousarray(np.asarray(list(seq) if not isinstance(seq, np.ndarray) else seq,
                                          dtype=np.int64))
    if arr.size and (arr.min() < -2**31 or arr.max() >= 2**31):
        raise ValueError("Token IDs must be in [0, vocab_size)")
    return np.ascontiguousarray(arr.astype(np.int32))


def inspect_checkpoint(directory, precision="bf16", strict=False):
    """Validate a converted checkpoint directory without the GPU; returns its
    architecture as a config dict."""
    cfg = ModelConfig()
    err = C.c_void_p()
    _check(lib.yuear_checkpoint_inspect(os.fsencode(directory), precision.encode(), int(strict),
                                        C.byref(cfg), C.byref(err)), err)
    return dict(hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                num_hidden_layers=cfg.num_hidden_layers,
                num_attention_heads=cfg.num_attention_heads,
                num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                vocab_size=cfg.vocab_size, max_position_embeddings=cfg.max_position_embeddings,
                rms_norm_eps=float(cfg.rms_norm_eps), rope_theta=float(cfg.rope_theta),
                qk_norm=bool(cfg.qk_norm))


class Engine:
    """ARModel equivalent: device weights for one config (ar.cpp:133-245)."""

    def __init__(self, config: dict, weights: dict | None = None, *, seed=0, std=0.02,
                 norm_std=0.0, bits=0):
        """bits 8 / 4: affine group-64 quantized linears (the "8bit" / "4bit"
        precisions): `weights` then holds uint32 codes for every `*_proj` /
        `lm_head` `.weight` plus bf16 `.scales` / `.biases`; without weights
        the random bf16 linears are quantized by `quantize_affine`."""
        self.config = dict(config)
        self._cfg = _config_struct(self.config)
        keep = []
        if weights is None:
            src = WeightSource(0, seed, std, norm_std, None, 0, bits)
        else:
            table = (TensorC * len(weights))()
            for i, (name, arr) in enumerate(weights.items()):
                u32 = np.asarray(arr).dtype == np.uint32
                arr = np.ascontiguousarray(arr, dtype=np.uint32 if u32 else np.uint16)
                keep.append(arr)
                table[i] = TensorC(name.encode(), arr.ctypes.data, arr.size,
                                   DTYPE_U32 if u32 else DTYPE_BF16)
            keep.append(table)
            src = WeightSource(1, 0, 0.0, 0.0, table, len(weights), bits)
        handle = C.c_void_p()
        err = C.c_void_p()
        _check(lib.yuear_engine_create(C.byref(self._cfg), C.byref(src), C.byref(handle),
                                       C.byref(err)), err)
        self.handle = handle

    @classmethod
    def load(cls, directory, precision="bf16", strict=False):
        """ARModel(directory, precision) (ar.cpp:133-238) from a converted
        checkpoint directory (conversion.json, config.json,
        ar-<precision>.safetensors)."""
        self = cls.__new__(cls)
        self.config = inspect_checkpoint(directory, precision, strict)
        self._cfg = _config_struct(self.config)
        handle = C.c_void_p()
        err = C.c_void_p()
        _check(lib.yuear_engine_load(os.fsencode(directory), precision.encode(), int(strict),
                                     C.byref(handle), C.byref(err)), err)
        self.handle = handle
        return self

    def close(self, _destroy=lib.yuear_engine_destroy):
        # _destroy is bound at definition: at interpreter exit the module's
        # globals may already be gone when __del__ runs
        if getattr(self, "handle", None):
            _destroy(self.handle)
            self.handle = None

    __del__ = close

    def cancel(self):
        lib.yuear_engine_cancel(self.handle)

    def nar_condition(self, tokens, visible_end=0):
        """CachedNAR's conditioning prefill (nar.cpp:139-190): per layer the keys
        and values of the visible prefix, as torch bf16 device tensors
        [layers, kv_heads, visible, 128] (plumbing; the work is libyuear's)."""
        import torch
        c = self.config
        ids = _i32(tokens)
        n = len(ids)
        visible = min(visible_end, n) if visible_end else n
        shape = (c["num_hidden_layers"], c["num_key_value_heads"], max(visible, 1), 128)
        k = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
        v = torch.empty_like(k)
        got = C.c_int32()
        err = C.c_void_p()
        _check(lib.yuear_nar_condition(self.handle, ids.ctypes.data_as(i32p), n, int(visible_end),
                                       k.data_ptr(), v.data_ptr(), C.byref(got), C.byref(err)),
               err)
        return k[:, :, :got.value], v[:, :, :got.value]

    @property
    def bits(self):
        """0 for bf16 linears, else the quantization bits."""
        return lib.yuear_engine_bits(self.handle)

    def session(self, branches=1, capacity=1024, phase="full"):
        return Session(self, branches, capacity, phase)

    def generate_tokens(self, prefix, sampling, seed, phase="full", negative=None, cfg_scale=1.0,
                        legacy_off=False, on_token=None, cancelled=None):
        """sampling.cpp:185-288 -> (tokens, timing, truncated). `cancelled`: a
        predicate polled where the reference calls cancelled_at (before each
        prefill, between prefill chunks, before each token); a cancelled run
        raises InterruptedError with the reference's message."""
        pre = _i32(prefix)
        neg = _i32(negative) if negative is not None else np.zeros(0, dtype=np.int32)
        s = sampling_struct(sampling)
        out = np.zeros(max(1, s.max_tokens), dtype=np.int32)
        n = C.c_int32()
        trunc = C.c_int32()
        timing = C.c_void_p()
        err = C.c_void_p()
        failure = []

        def _cb(_user, phase_bytes, token):
            if on_token is None:
                return
            try:
                on_token(phase_bytes.decode(), int(token))
            except BaseException as exc:  # a throwing callback cancels (runtime.mm:143-186)
                failure.append(exc)
                self.cancel()

        def _poll(_user):
            if failure:
                return 1
            try:
                return 1 if cancelled is not None and cancelled() else 0
            except BaseException as exc:  # a throwing predicate cancels too
                failure.append(exc)
                return 1

        cb = TOKEN_CB(_cb)
        poll = CANCEL_POLL(_poll) if cancelled is not None else CANCEL_POLL()
        status = lib.yuear_generate_tokens(
            self.handle, pre.ctypes.data_as(i32p), pre.size, C.byref(s), int(seed),
            phase.encode(), neg.ctypes.data_as(i32p) if neg.size else None, neg.size,
            float(cfg_scale), int(legacy_off), poll, cb, None, out.ctypes.data_as(i32p),
            C.byref(n),
            C.byref(trunc), C.byref(timing), C.byref(err))
        if failure:
            if err.value:
                lib.yuear_string_free(err)
            raise failure[0]
        _check(status, err)
        text = C.cast(timing, C.c_char_p).value.decode()
        lib.yuear_string_free(timing)
        return out[:n.value].tolist(), json.loads(text), bool(trunc.value)


class Session:
    """Fixed-capacity decode session: GraphAR semantics (cuda_graph.py:43-240)."""

    def __init__(self, engine: Engine, branches, capacity, phase="full"):
        self.engine = engine
        self.branches = branches
        self.capacity = capacity
        handle = C.c_void_p()
        err = C.c_void_p()
        _check(lib.yuear_session_begin(engine.handle, branches, capacity, phase.encode(),
                                       C.byref(handle), C.byref(err)), err)
        self.handle = handle
        self.vocab = lib.yuear_session_phase_size(handle)

    def close(self, _end=lib.yuear_session_end):
        if getattr(self, "handle", None):
            _end(self.handle)
            self.handle = None

    __del__ = close

    def _h(self):
        if not self.handle:
            raise RuntimeError("session is closed")
        return self.handle

    def position(self, branch=0):
        return lib.yuear_session_position(self._h(), branch)

    def prefill(self, branch, ids):
        ids = _i32(ids)
        logits = np.empty(self.vocab, dtype=np.uint16)
        err = C.c_void_p()
        _check(lib.yuear_session_prefill(self._h(), branch, ids.ctypes.data_as(i32p), ids.size,
                                         logits.ctypes.data_as(u16p), C.byref(err)), err)
        return logits

    def step(self, tokens):
        if np.isscalar(tokens):
            tokens = [int(tokens)] * self.branches
        tokens = _i32(tokens)
        if tokens.size != self.branches:
            raise ValueError("step needs one token per branch")
        logits = np.empty((self.branches, self.vocab), dtype=np.uint16)
        err = C.c_void_p()
        _check(lib.yuear_session_step(self._h(), tokens.ctypes.data_as(i32p),
                                      logits.ctypes.data_as(u16p), C.byref(err)), err)
        return logits

    def sample(self, sampling, seed, step, history=(), cfg_scale=1.0, legacy_off=False):
        s = sampling_struct(sampling)
        hist = _i32(history)
        tok = C.c_int32()
        err = C.c_void_p()
        _check(lib.yuear_session_sample(self._h(), C.byref(s), int(seed), float(cfg_scale),
                                        int(legacy_off), int(step),
                                        hist.ctypes.data_as(i32p) if hist.size else None,
                                        hist.size, C.byref(tok), C.byref(err)), err)
        return int(tok.value)

    def write_kv(self, layer, branch, keys, values):
        """keys/values [Hkv, n, D] bf16 -> slots [0, n); position becomes n."""
        k = np.ascontiguousarray(keys, dtype=np.uint16)
        v = np.ascontiguousarray(values, dtype=np.uint16)
        err = C.c_void_p()
        _check(lib.yuear_session_write_kv(self._h(), layer, branch, k.ctypes.data_as(u16p),
                                          v.ctypes.data_as(u16p), k.shape[1], C.byref(err)), err)

    def read_kv(self, layer, branch, n):
        c = self.engine.config
        shape = (c["num_key_value_heads"], n, c["head_dim"])
        k = np.empty(shape, dtype=np.uint16)
        v = np.empty(shape, dtype=np.uint16)
        err = C.c_void_p()
        _check(lib.yuear_session_read_kv(self._h(), layer, branch, k.ctypes.data_as(u16p),
                                         v.ctypes.data_as(u16p), n, C.byref(err)), err)
        return k, v

    def write_logits(self, logits):
        arr = np.ascontiguousarray(logits, dtype=np.uint16).reshape(self.branches, self.vocab)
        err = C.c_void_p()
        _check(lib.yuear_session_write_logits(self._h(), arr.ctypes.data_as(u16p), C.byref(err)),
               err)

    def set_position(self, branch, position):
        err = C.c_void_p()
        _check(lib.yuear_session_set_position(self._h(), branch, position, C.byref(err)), err)

    def layer_step(self, layer, x):
        x = np.ascontiguousarray(x, dtype=np.uint16).reshape(self.branches, -1)
        out = np.empty_like(x)
        err = C.c_void_p()
        _check(lib.yuear_session_layer_step(self._h(), layer, x.ctypes.data_as(u16p),
                                            out.ctypes.data_as(u16p), C.byref(err)), err)
        return out

    def time_generate(self, sampling, seed, steps, reset=True):
        """(ms per token, emitted native ids) of `steps` device-side decode
        iterations (sampler -> step graph replays, no host sync between)."""
        s = sampling_struct(sampling)
        ms = C.c_double()
        out = np.zeros(steps, dtype=np.int32)
        err = C.c_void_p()
        _check(lib.yuear_session_time_generate(self._h(), C.byref(s), int(seed), steps,
                                               int(reset), C.byref(ms),
                                               out.ctypes.data_as(i32p), C.byref(err)), err)
        return ms.value, out.tolist()

    def time_kernel(self, kernel, launches):
        ms = C.c_double()
        err = C.c_void_p()
        _check(lib.yuear_session_time_kernel(self._h(), kernel.encode(), launches, C.byref(ms),
                                             C.byref(err)), err)
        return ms.value

    def time_steps(self, steps):
        ms = C.c_double()
        err = C.c_void_p()
        _check(lib.yuear_session_time_steps(self._h(), steps, C.byref(ms), C.byref(err)), err)
        return ms.value


# ---- text side of a request (host only, no GPU): protocol.hpp / protocol.mm ----

def _ids_out(ptr, n):
    ids = [ptr[i] for i in range(n.value)]
    lib.yuear_ids_free(ptr)
    return ids


def _ids_in(ids):
    arr = np.ascontiguousarray(np.asarray(list(ids) if ids is not None else [], dtype=np.int32))
    return arr, arr.ctypes.data_as(i32p)


class Tokenizer:
    """lyra::Tokenizer (protocol.hpp:5-16): ``encode(text) -> ids`` and
    ``decode(ids) -> text`` over a checkpoint-native qwen.tiktoken."""

    def __init__(self, vocabulary):
        self._t = C.c_void_p()
        err = C.c_void_p()
        _check(lib.yuear_tokenizer_load(os.fsencode(vocabulary), C.byref(self._t), C.byref(err)),
               err)

    def close(self, _destroy=lib.yuear_tokenizer_destroy):
        if getattr(self, "_t", None):
            _destroy(self._t)
            self._t = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, text):
        data = text.encode("utf-8", errors="surrogatepass") if isinstance(text, str) else bytes(text)
        ptr, n, err = i32p(), C.c_int64(), C.c_void_p()
        _check(lib.yuear_tokenizer_encode(self._t, data, len(data), C.byref(ptr), C.byref(n),
                                          C.byref(err)), err)
        return _ids_out(ptr, n)

    def decode(self, ids):
        arr, p = _ids_in(ids)
        out, n, err = C.c_void_p(), C.c_int64(), C.c_void_p()
        _check(lib.yuear_tokenizer_decode(self._t, p, arr.size, C.byref(out), C.byref(n),
                                          C.byref(err)), err)
        text = C.string_at(out, n.value).decode("utf-8")
        lib.yuear_string_free(out)
        return text


def text_nfc(text):
    """Test hook: the library's NFC of `text` (str or UTF-8 bytes)."""
    data = text.encode("utf-8", errors="surrogatepass") if isinstance(text, str) else bytes(text)
    out, n, err = C.c_void_p(), C.c_int64(), C.c_void_p()
    _check(lib.yuear_text_nfc(data, len(data), C.byref(out), C.byref(n), C.byref(err)), err)
    value = C.string_at(out, n.value).decode("utf-8")
    lib.yuear_string_free(out)
    return value


def text_pieces(text):
    """Test hook: the pre-tokenizer's pieces (str) of the NFC form of `text`."""
    data = text.encode("utf-8", errors="surrogatepass") if isinstance(text, str) else bytes(text)
    ptr, n, err = i32p(), C.c_int64(), C.c_void_p()
    _check(lib.yuear_text_pieces(data, len(data), C.byref(ptr), C.byref(n), C.byref(err)), err)
    ends = _ids_out(ptr, n)
    nfc = text_nfc(data).encode("utf-8")
    return [nfc[a:b].decode("utf-8") for a, b in zip([0] + ends[:-1], ends)]


class SongRequest:
    """The SongRequest fields the prompt layout reads (types.hpp:50-62;
    defaults cot "full", seed 831001, id "song")."""

    def __init__(self, style, lyrics, cot="full", seed=831001, abc=None, cfg_scale=None,
                 id="song"):
        self.style, self.lyrics, self.cot, self.seed = style, lyrics, cot, seed
        self.abc, self.cfg_scale, self.id = abc, cfg_scale, id

    def _c(self):
        enc = (lambda v: None if v is None else v.encode("utf-8"))
        return SongRequestC(enc(self.style), enc(self.lyrics), enc(self.cot), enc(self.abc),
                            enc(self.id), int(self.seed),
                            0.0 if self.cfg_scale is None else float(self.cfg_scale),
                            int(self.cfg_scale is not None))

    def validate(self):
        err = C.c_void_p()
        r = self._c()
        _check(lib.yuear_song_request_validate(C.byref(r), C.byref(err)), err)

    @property
    def guidance(self):
        r = self._c()
        return lib.yuear_song_request_guidance(C.byref(r))


def _prefix(fn, tokenizer, request, abc_ids):
    arr, p = _ids_in(abc_ids)
    r = request._c()
    ptr, n, err = i32p(), C.c_int64(), C.c_void_p()
    _check(fn(tokenizer._t, C.byref(r), p, arr.size, int(abc_ids is not None), C.byref(ptr),
              C.byref(n), C.byref(err)), err)
    return _ids_out(ptr, n)


def token_prefixes(request, tokenizer, abc_ids=None):
    """token_prefixes (protocol.mm:321-340)."""
    return _prefix(lib.yuear_token_prefixes, tokenizer, request, abc_ids)


def negative_prefix(request, tokenizer, abc_ids=None):
    """negative_prefix (protocol.mm:341-357)."""
    return _prefix(lib.yuear_negative_prefix, tokenizer, request, abc_ids)


def chunk_ranges(frames, prefix_tokens, context=24576):
    """chunk_ranges (protocol.mm:358-369): [(a, b), ...] frame chunks."""
    ptr, n, err = i32p(), C.c_int64(), C.c_void_p()
    _check(lib.yuear_chunk_ranges(int(frames), int(prefix_tokens), int(context), C.byref(ptr),
                                  C.byref(n), C.byref(err)), err)
    flat = [ptr[i] for i in range(2 * n.value)]
    lib.yuear_ids_free(ptr)
    return list(zip(flat[0::2], flat[1::2]))
