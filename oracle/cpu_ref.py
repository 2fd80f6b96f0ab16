"""ctypes wrapper of the CPU oracle (oracle/liboracle.so). TEST INFRASTRUCTURE.

Only tests, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` import this module. bf16 arrays are numpy ``uint16`` bit
patterns throughout.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

PHASES = {"full": 0, "abc": 1, "semantic": 2}

u16p = C.POINTER(C.c_uint16)
i32p = C.POINTER(C.c_int32)
u32p = C.POINTER(C.c_uint32)
f32p = C.POINTER(C.c_float)


class Config(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("intermediate", C.c_int32), ("layers", C.c_int32),
                ("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("vocab", C.c_int32), ("rms_eps", C.c_float), ("rope_theta", C.c_double),
                ("qk_norm", C.c_int32)]


class Weights(C.Structure):
    _fields_ = [(name, u16p) for name in ("embed", "final_norm", "lm_head")] + [
        (name, C.POINTER(u16p)) for name in
        ("input_ln", "post_ln", "q_norm", "k_norm", "wq", "wk", "wv", "wo", "wg", "wu", "wd")]


LINEARS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
           "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


class Quant(C.Structure):
    _fields_ = [("bits", C.c_int32), ("lm_scales", u16p), ("lm_biases", u16p),
                ("scales", C.POINTER(u16p) * 7), ("biases", C.POINTER(u16p) * 7)]


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_double), ("top_p", C.c_double), ("top_k", C.c_int32),
                ("repetition_penalty", C.c_double), ("penalty_window", C.c_int32),
                ("min_tokens", C.c_int32), ("max_tokens", C.c_int32)]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    sig = {
        "oracle_f2bf": (C.c_uint16, [C.c_float]),
        "oracle_bf2f": (C.c_float, [C.c_uint16]),
        "oracle_philox4x32_10": (None, [C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                        C.POINTER(C.c_uint32)]),
        "oracle_uniform": (C.c_float, [C.c_uint64, C.c_int32, C.c_int32]),
        "oracle_plog": (C.c_float, [C.c_float]),
        "oracle_pexp": (C.c_float, [C.c_float]),
        "oracle_set_threads": (None, [C.c_int]),
        "oracle_set_accumulation": (None, [C.c_int]),
        "oracle_rms_norm": (None, [u16p, C.c_int, C.c_int, u16p, C.c_float, u16p]),
        "oracle_linear": (None, [u16p, C.c_int, C.c_int, u16p, C.c_int, u16p]),
        "oracle_rope": (None, [u16p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double]),
        "oracle_rope_table": (None, [C.c_int, C.c_int, C.c_double, u16p, u16p]),
        "oracle_silu_mul": (None, [u16p, u16p, C.c_int, u16p]),
        "oracle_attention": (None, [u16p, u16p, u16p, C.c_int, C.c_int, C.c_int, C.c_int,
                                    C.c_int, C.c_int, u16p]),
        "oracle_nar_attention": (None, [u16p, u16p, u16p, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.c_int, C.c_int, C.c_int, u16p]),
        "oracle_model_new": (C.c_void_p, [C.POINTER(Config), C.POINTER(Weights)]),
        "oracle_model_new_quantized": (C.c_void_p, [C.POINTER(Config), C.POINTER(Weights),
                                                    C.POINTER(Quant)]),
        "oracle_qlinear": (None, [u16p, C.c_int, C.c_int, u32p, u16p, u16p, C.c_int, C.c_int,
                                  u16p]),
        "oracle_dequantize": (None, [u32p, u16p, u16p, C.c_int, C.c_int, C.c_int, u16p]),
        "oracle_model_free": (None, [C.c_void_p]),
        "oracle_cache_new": (C.c_void_p, [C.c_void_p, C.c_int]),
        "oracle_cache_free": (None, [C.c_void_p]),
        "oracle_cache_offset": (C.c_int, [C.c_void_p]),
        "oracle_cache_set_offset": (None, [C.c_void_p, C.c_int]),
        "oracle_cache_capacity": (C.c_int, [C.c_void_p]),
        "oracle_cache_keys": (u16p, [C.c_void_p, C.c_int]),
        "oracle_cache_values": (u16p, [C.c_void_p, C.c_int]),
        "oracle_layer": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, u16p, C.c_int]),
        "oracle_hidden": (C.c_int, [C.c_void_p, C.c_void_p, i32p, C.c_int, u16p]),
        "oracle_project": (C.c_int, [C.c_void_p, u16p, C.c_int, u16p]),
        "oracle_phase_size": (C.c_int, [C.c_void_p, C.c_int]),
        "oracle_guided_logits": (None, [u16p, u16p, C.c_int, C.c_double, u16p]),
        "oracle_distribution": (C.c_int, [u16p, C.c_int, C.POINTER(Sampling), i32p, C.c_int,
                                          C.c_int, C.c_int, C.c_int, f32p]),
        "oracle_draw": (C.c_int, [f32p, C.c_int, C.c_double, C.c_uint64, C.c_int]),
        "oracle_native_to_local": (C.c_int, [C.c_int, C.c_int, C.c_int]),
        "oracle_local_to_native": (C.c_int, [C.c_int, C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


# ---- numpy bf16 helpers (the oracle's own RNE, vectorised) ----

def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _u16(a):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    return a, a.ctypes.data_as(u16p)


# ---- model_ops ----

def rms_norm(x, w, eps):
    x, px = _u16(x)
    w, pw = _u16(w)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().oracle_rms_norm(px, x.size // n, n, pw, eps, y.ctypes.data_as(u16p))
    return y


def linear(x, w):
    x, px = _u16(x)
    w, pw = _u16(w)
    n, k = w.shape
    y = np.empty(x.shape[:-1] + (n,), dtype=np.uint16)
    lib().oracle_linear(px, x.size // k, k, pw, n, y.ctypes.data_as(u16p))
    return y


def qlinear(x, wq, scales, biases, bits):
    """Affine group-64 quantized linear: wq [n][k * bits / 32] uint32 codes,
    scales / biases [n][k / 64] bf16."""
    x, px = _u16(x)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales, ps = _u16(scales)
    biases, pb = _u16(biases)
    n, k = scales.shape[0], scales.shape[1] * 64
    y = np.empty(x.shape[:-1] + (n,), dtype=np.uint16)
    lib().oracle_qlinear(px, x.size // k, k, wq.ctypes.data_as(u32p), ps, pb, bits, n,
                         y.ctypes.data_as(u16p))
    return y


def dequantize(wq, scales, biases, bits):
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales, ps = _u16(scales)
    biases, pb = _u16(biases)
    n, k = scales.shape[0], scales.shape[1] * 64
    out = np.empty((n, k), dtype=np.uint16)
    lib().oracle_dequantize(wq.ctypes.data_as(u32p), ps, pb, bits, n, k, out.ctypes.data_as(u16p))
    return out


def rope(x, offset, theta):
    """x [T, heads, D] bf16 -> rotated copy."""
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    T, heads, d = x.shape
    lib().oracle_rope(x.ctypes.data_as(u16p), T, heads, d, offset, theta)
    return x


def rope_table(positions, d, theta):
    c = np.empty((positions, d // 2), dtype=np.uint16)
    s = np.empty_like(c)
    lib().oracle_rope_table(positions, d, theta, c.ctypes.data_as(u16p), s.ctypes.data_as(u16p))
    return c, s


def silu_mul(g, u):
    g, pg = _u16(g)
    u, pu = _u16(u)
    out = np.empty_like(g)
    lib().oracle_silu_mul(pg, pu, g.size, out.ctypes.data_as(u16p))
    return out


def attention(q, keys, values, offset):
    """q [T, Hq, D]; keys/values [Hkv, cap, D] -> [T, Hq*D]."""
    q, pq = _u16(q)
    keys, pk = _u16(keys)
    values, pv = _u16(values)
    T, Hq, D = q.shape
    Hkv, cap, _ = keys.shape
    out = np.empty((T, Hq * D), dtype=np.uint16)
    lib().oracle_attention(pq, pk, pv, T, Hq, Hkv, D, cap, offset, out.ctypes.data_as(u16p))
    return out


def nar_attention(q, keys, values, causal=False):
    """q [B, Hq, Lq, D]; keys/values [B, Hkv, Lk, D] -> [B, Hq, Lq, D]
    (nar_attention.cpp:63-270)."""
    q, pq = _u16(q)
    keys, pk = _u16(keys)
    values, pv = _u16(values)
    B, Hq, Lq, D = q.shape
    _, Hkv, Lk, _ = keys.shape
    out = np.empty_like(q)
    lib().oracle_nar_attention(pq, pk, pv, B, Hq, Hkv, Lq, Lk, D, int(causal),
                               out.ctypes.data_as(u16p))
    return out


def philox(ctr, key):
    c = (C.c_uint32 * 4)(*ctr)
    k = (C.c_uint32 * 2)(*key)
    o = (C.c_uint32 * 4)()
    lib().oracle_philox4x32_10(c, k, o)
    return [int(v) for v in o]


def guided_logits(c, u, scale):
    c, pc = _u16(c)
    u, pu = _u16(u)
    out = np.empty_like(c)
    lib().oracle_guided_logits(pc, pu, c.size, scale, out.ctypes.data_as(u16p))
    return out


def sampling_struct(temperature=1.0, top_p=0.95, top_k=100, repetition_penalty=1.2,
                    penalty_window=50, min_tokens=200, max_tokens=9000):
    return Sampling(temperature, top_p, top_k, repetition_penalty, penalty_window,
                    min_tokens, max_tokens)


def distribution(logits, sampling, history, step, phase="full", legacy_off=False):
    logits, pl = _u16(logits)
    hist = np.ascontiguousarray(np.asarray(history, dtype=np.int32))
    scores = np.empty(logits.size, dtype=np.float32)
    rc = lib().oracle_distribution(pl, logits.size, C.byref(sampling),
                                   hist.ctypes.data_as(i32p), hist.size, step,
                                   PHASES[phase], int(legacy_off), scores.ctypes.data_as(f32p))
    if rc:
        raise ValueError("Incorrect projected phase vocabulary size")
    return scores


def draw(scores, temperature, seed, step):
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    return lib().oracle_draw(scores.ctypes.data_as(f32p), scores.size, temperature, seed, step)


# ---- model ----

LAYER_TENSORS = [("input_ln", "input_layernorm"), ("post_ln", "post_attention_layernorm"),
                 ("q_norm", "self_attn.q_norm"), ("k_norm", "self_attn.k_norm"),
                 ("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"),
                 ("wv", "self_attn.v_proj"), ("wo", "self_attn.o_proj"),
                 ("wg", "mlp.gate_proj"), ("wu", "mlp.up_proj"), ("wd", "mlp.down_proj")]


class Model:
    """Oracle ARModel over host weights keyed by the reference tensor names."""

    def __init__(self, config: dict, weights: dict, bits: int = 0):
        """bits 8 / 4: the projections and lm_head are affine group-64 quantized
        (``<name>.weight`` uint32 codes, ``<name>.scales`` / ``<name>.biases`` bf16)."""
        self.config = dict(config)
        self.bits = bits
        self.weights = {k: np.ascontiguousarray(v, dtype=np.uint32 if v.dtype == np.uint32
                                                else np.uint16) for k, v in weights.items()}
        c = self.config
        self._cfg = Config(c["hidden_size"], c["intermediate_size"], c["num_hidden_layers"],
                           c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"],
                           c["vocab_size"], c["rms_norm_eps"], c["rope_theta"],
                           int(c.get("qk_norm", True)))
        L = c["num_hidden_layers"]
        w = self.weights
        self._arrays = {}
        fields = {}
        for field, suffix in LAYER_TENSORS:
            arr = (u16p * L)(*[w[f"model.layers.{i}.{suffix}.weight"].ctypes.data_as(u16p)
                               for i in range(L)])
            self._arrays[field] = arr
            fields[field] = C.cast(arr, C.POINTER(u16p))
        self._w = Weights(w["model.embed_tokens.weight"].ctypes.data_as(u16p),
                          w["model.norm.weight"].ctypes.data_as(u16p),
                          w["lm_head.weight"].ctypes.data_as(u16p), **fields)
        if bits:
            def table(suffix):
                arr = (u16p * L)(*[w[f"model.layers.{i}.{suffix}"].ctypes.data_as(u16p)
                                   for i in range(L)])
                self._arrays[suffix] = arr
                return C.cast(arr, C.POINTER(u16p))
            self._q = Quant(bits, w["lm_head.scales"].ctypes.data_as(u16p),
                            w["lm_head.biases"].ctypes.data_as(u16p),
                            (C.POINTER(u16p) * 7)(*[table(n + ".scales") for n in LINEARS]),
                            (C.POINTER(u16p) * 7)(*[table(n + ".biases") for n in LINEARS]))
            self.handle = lib().oracle_model_new_quantized(C.byref(self._cfg), C.byref(self._w),
                                                           C.byref(self._q))
        else:
            self.handle = lib().oracle_model_new(C.byref(self._cfg), C.byref(self._w))
        if not self.handle:
            raise ValueError("invalid oracle model configuration")

    def __del__(self):
        if getattr(self, "handle", None):
            lib().oracle_model_free(self.handle)
            self.handle = None

    def cache(self, capacity):
        return Cache(self, capacity)

    def hidden(self, ids, cache):
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        out = np.empty((ids.size, self.config["hidden_size"]), dtype=np.uint16)
        rc = lib().oracle_hidden(self.handle, cache.handle, ids.ctypes.data_as(i32p), ids.size,
                                 out.ctypes.data_as(u16p))
        if rc:
            raise ValueError("KV cache capacity exceeded or invalid token ids")
        return out

    def layer(self, index, x, cache):
        x = np.array(x, dtype=np.uint16, copy=True, order="C")
        rc = lib().oracle_layer(self.handle, cache.handle, index, x.ctypes.data_as(u16p),
                                x.shape[0])
        if rc:
            raise ValueError("KV cache capacity exceeded")
        return x

    def phase_size(self, phase):
        return lib().oracle_phase_size(self.handle, PHASES[phase])

    def project(self, h, phase="full"):
        h, ph = _u16(h)
        out = np.empty(self.phase_size(phase), dtype=np.uint16)
        if lib().oracle_project(self.handle, ph, PHASES[phase], out.ctypes.data_as(u16p)):
            raise ValueError("phase must be 'abc' or 'semantic'")
        return out

    def prefill(self, ids, cache, phase="full", chunk=1024):
        """sampling.cpp:152-183: chunked hidden(), logits of the last token."""
        h = None
        for start in range(0, len(ids), chunk):
            h = self.hidden(ids[start:start + chunk], cache)
        return self.project(h[-1], phase)

    def step(self, token, cache, phase="full"):
        return self.project(self.hidden([token], cache)[-1], phase)


class Cache:
    def __init__(self, model: Model, capacity: int):
        self.model = model
        self.handle = lib().oracle_cache_new(model.handle, capacity)
        if not self.handle:
            raise ValueError("KV cache capacity must be in [1, 24576]")
        c = model.config
        self.shape = (c["num_key_value_heads"], capacity, c["head_dim"])

    def __del__(self):
        if getattr(self, "handle", None):
            lib().oracle_cache_free(self.handle)
            self.handle = None

    @property
    def offset(self):
        return lib().oracle_cache_offset(self.handle)

    @offset.setter
    def offset(self, value):
        lib().oracle_cache_set_offset(self.handle, value)

    def keys(self, layer):
        """Writable numpy view [Hkv, cap, D] of one layer's key storage."""
        p = lib().oracle_cache_keys(self.handle, layer)
        return np.ctypeslib.as_array(p, shape=self.shape)

    def values(self, layer):
        p = lib().oracle_cache_values(self.handle, layer)
        return np.ctypeslib.as_array(p, shape=self.shape)
