"""The attention kernels' P split, restated on the CPU (float32 numpy).

Each softmax weight p = exp2(s - m) in (0, 1] is split into three bf16
pieces so that the MFMA's bf16 products V * piece carry all of p:

- the prefill / acoustic-model tile (attn_tile.h) truncates: hi keeps the
  top 8 significant bits of p, mid the top 8 of p - hi, lo the rest;
- the decode pass (attn_core.h) rounds each piece to nearest even
  (integer form, f2bf_int).

Both are exact when the pieces sum back to p: every remainder is exactly
representable, so p - hi and p - hi - mid carry no rounding. This test
checks that, that each piece is a bf16 value, and that V * piece for a bf16
V is exact in fp32 (8 x 8 significant bits), over edge cases and random
exponents, for normal fp32 p (p >= 2^-126; smaller weights are below the
fp32 result's resolution next to the maximum term, which is 1): exact for
p >= 2^-102, where every remainder is a normal fp32 number; below that, what
the three pieces miss is under 2^-126 in absolute terms.
"""
import numpy as np
import pytest


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def f32(u):
    return np.asarray(u, np.uint32).view(np.float32)


def split_truncate(p):
    """attn_tile.h: pw[k] = high half of the remainder, remainder -= it."""
    p = np.asarray(p, np.float32).copy()
    pieces = []
    for _ in range(3):
        hi = f32(bits(p) & np.uint32(0xFFFF0000))
        pieces.append(hi)
        p = (p - hi).astype(np.float32)
    return pieces, p


def f2bf_int(x):
    """common.h f2bf_int: round to nearest even on the bit pattern."""
    u = bits(x).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return r.astype(np.uint32)


def split_rne(p):
    """attn_core.h: b = f2bf_int(rem), rem -= bf2f(b)."""
    p = np.asarray(p, np.float32).copy()
    pieces = []
    for _ in range(3):
        b = f2bf_int(p)
        piece = f32(b << np.uint32(16))
        pieces.append(piece)
        p = (p - piece).astype(np.float32)
    return pieces, p


def weights(rng, n):
    # exp2 of (s - m) <= 0 over the normal range, plus edge cases
    e = -rng.uniform(0.0, 126.0, size=n).astype(np.float32)
    p = np.exp2(e).astype(np.float32)
    edge = np.array([1.0, np.nextafter(np.float32(1.0), np.float32(0.0)), 0.5, 2.0 ** -126,
                     np.float32(2.0 ** -126) * np.float32(1.9999999), 1.0 - 2.0 ** -8,
                     1.0 - 2.0 ** -9, 1.0 + 0.0, 0.99609375, 0.998046875,
                     f32(np.uint32(0x3F7FFFFF)), f32(np.uint32(0x3F7F8000)),
                     f32(np.uint32(0x3F7F7FFF)), f32(np.uint32(0x3F008001))], np.float32)
    # every 24-bit significand pattern class: hi / mid / lo bits set or not
    sig = rng.integers(0, 1 << 23, size=n // 4, dtype=np.uint32)
    pat = f32((np.uint32(126) << np.uint32(23)) | sig)  # [0.5, 1)
    return np.concatenate([p, edge, pat])


@pytest.mark.parametrize("split", [split_truncate, split_rne], ids=["truncate", "rne"])
def test_split_is_exact(split):
    rng = np.random.default_rng(5)
    p = weights(rng, 1_000_000)
    pieces, rest = split(p)
    for piece in pieces:  # bf16 values: the low half of the pattern is zero
        assert (bits(piece) & np.uint32(0xFFFF)).max() == 0
    big = p >= np.float32(2.0 ** -102)
    assert big.mean() > 0.7
    np.testing.assert_array_equal(rest[big], 0.0)  # nothing left after three pieces
    total = sum(x.astype(np.float64) for x in pieces)
    np.testing.assert_array_equal(total[big], p[big].astype(np.float64))
    assert np.abs(total - p.astype(np.float64)).max() < 2.0 ** -126
    # V * piece exact in fp32 for bf16 V: compare against the float64 product
    v = f32(bits(rng.normal(size=p.size).astype(np.float32)) & np.uint32(0xFFFF0000))
    for piece in pieces:
        prod64 = v.astype(np.float64) * piece.astype(np.float64)
        normal = np.abs(prod64) >= 2.0 ** -126  # products that do not underflow
        prod32 = (v * piece).astype(np.float32).astype(np.float64)
        np.testing.assert_array_equal(prod32[normal], prod64[normal])


def test_truncate_and_rne_pieces_differ_but_sum_the_same():
    # 1 - 2^-9 truncates to 0.99609375 + ... but rounds to 1.0 - ...: the
    # pieces differ (the RNE remainder is negative), the sums are both p
    p = np.array([1.0 - 2.0 ** -9], np.float32)
    t, _ = split_truncate(p)
    r, _ = split_rne(p)
    assert t[0][0] == np.float32(0.99609375) and r[0][0] == np.float32(1.0)
    assert r[1][0] < 0
    assert sum(float(x[0]) for x in t) == sum(float(x[0]) for x in r) == float(p[0])
