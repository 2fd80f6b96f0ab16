"""Affine group-64 quantized tensors for the tests (the layout of the
reference's quantized checkpoints, native/src/conversion.cpp:287-300,
470-532: `<name>.weight` uint32 [rows][k * bits / 32], `<name>.scales` and
`<name>.biases` bf16 [rows][k / 64]; dequantized value s * q + b).

Codes are drawn directly (uniform), not produced by a quantizer, so nothing
here depends on how a converter picks scales. `unpack_bytes` recovers the
codes through a little-endian byte view of the words, a route independent of
the word shifts the oracle and the kernels use.
"""
import numpy as np

LINEARS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
           "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


def pack(codes, bits):
    """codes [rows][k] (values < 2**bits) -> uint32 words, code j of a word at
    bits [bits * j, bits * j + bits)."""
    codes = np.asarray(codes, dtype=np.uint32)
    per = 32 // bits
    rows, k = codes.shape
    c = codes.reshape(rows, k // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * bits)[None, None, :]
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def unpack_bytes(words, bits):
    """Inverse of `pack` through the byte view (little-endian words)."""
    b = np.ascontiguousarray(words, dtype="<u4").view(np.uint8).reshape(words.shape[0], -1)
    if bits == 8:
        return b.astype(np.int64)
    out = np.empty((b.shape[0], b.shape[1] * 2), dtype=np.int64)
    out[:, 0::2] = b & 0x0F
    out[:, 1::2] = b >> 4
    return out


def random_quantized(rng, rows, k, bits, std=0.02):
    """(words, scales, biases, codes) of a random [rows][k] matrix whose
    dequantized values have roughly the given standard deviation."""
    levels = (1 << bits) - 1
    codes = rng.integers(0, levels + 1, size=(rows, k), dtype=np.int64)
    step = std * np.sqrt(12.0) / levels
    scales = bf(step * rng.uniform(0.5, 1.5, size=(rows, k // 64)))
    biases = bf(-(levels / 2.0) * step * rng.uniform(0.8, 1.2, size=(rows, k // 64)))
    return pack(codes, bits), scales, biases, codes


def dequantize_f64(codes, scales, biases):
    import cpu_ref
    s = np.repeat(cpu_ref.bf16_to_f32(scales).astype(np.float64), 64, axis=1)
    b = np.repeat(cpu_ref.bf16_to_f32(biases).astype(np.float64), 64, axis=1)
    return s * codes + b


def quantize_model(weights, bits, seed=0):
    """Replace every projection and the lm_head of a bf16 weight dict by
    random quantized tensors of the same shape (norms and embedding stay
    bf16, linear_only=True). Returns the new dict."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, value in weights.items():
        base = name[:-len(".weight")] if name.endswith(".weight") else None
        if base and (base == "lm_head" or base.endswith(LINEARS)):
            rows, k = value.shape
            w, s, b, _ = random_quantized(rng, rows, k, bits)
            out[name], out[base + ".scales"], out[base + ".biases"] = w, s, b
        else:
            out[name] = value
    return out
