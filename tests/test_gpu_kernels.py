"""HIP kernels vs the oracle through the C ABI (op-level entry points).

Device memory comes from torch (plumbing only); every computation under test
runs in libyuear's gfx950 kernels. Tolerances (conftest.assert_close_bf16):
bf16 results of fp32 accumulations may differ from the oracle's by one unit
of the last place of the operands' scale when the two accumulation orders
round differently; most elements must be bit-identical.
"""
import numpy as np
import pytest

from conftest import assert_close_bf16, ulps_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    t.cuda.init()
    return t


def dev(torch, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def host(torch, t):
    torch.cuda.synchronize()
    out = t.cpu().numpy()
    return out.view(np.uint16) if out.dtype == np.int16 else out


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


def f(b):
    import cpu_ref
    return cpu_ref.bf16_to_f32(b)


GEMV_CASES = [  # (n, k, batch, norm, epilogue)
    (5120, 3072, 1, True, 0),     # fused QKV + input RMSNorm
    (3072, 3072, 1, False, 1),    # o_proj + residual
    (16384, 3072, 1, True, 2),    # gate/up interleaved + SwiGLU
    (3072, 8192, 1, False, 1),    # down + residual
    (83968, 3072, 1, True, 0),    # lm_head + final norm
    (5120, 3072, 2, True, 0),     # CFG pair
    (3072, 8192, 2, False, 1),
    (16384, 3072, 2, True, 2),
    (1024, 3072, 8, True, 0),     # batched sequences
    (1024, 8192, 8, False, 1),
    (1000, 256, 3, True, 0),      # ragged: odd batch, short rows, n % 8 != 0
    # 3..8 rows: MFMA form (hidden 3072 and 2048 layer shapes)
    (5120, 3072, 5, True, 0),
    (3072, 3072, 4, False, 1),
    (16384, 3072, 8, True, 2),
    (3072, 8192, 6, False, 1),
    (4096, 2048, 3, True, 0),
    (12288, 2048, 7, True, 2),
    (2048, 6144, 8, False, 1),
    (1000, 3072, 3, True, 0),     # n % 16 != 0
    (998, 3072, 5, True, 2),
    (5110, 3072, 8, False, 0),    # last 16-row block partly past n
    (4100, 3072, 3, True, 1),     # 257 blocks: one past a 256-CU grid, residual epilogue
    (2048, 6144, 4, True, 0),     # 16-wave forms with the RMSNorm prologue
    (1024, 8192, 8, True, 2),
    (96, 512, 1, False, 2),
]


@pytest.mark.parametrize("n,k,batch,norm,epilogue", GEMV_CASES)
def test_gemv_matches_oracle(torch, yuear_lib, oracle, n, k, batch, norm, epilogue):
    rng = np.random.default_rng(n + k + batch)
    w = bf(rng.normal(size=(n, k)) * 0.02)
    x = bf(rng.normal(size=(batch, k)))
    g = bf(1 + rng.normal(size=k) * 0.1)
    out_n = n // 2 if epilogue == 2 else n
    y0 = bf(rng.normal(size=(batch, out_n)))
    h = oracle.rms_norm(x, g, 1e-5) if norm else x
    acc = oracle.linear(h, w)
    if epilogue == 0:
        ref = acc
    elif epilogue == 1:
        ref = bf(f(y0) + f(acc))
    else:
        ref = oracle.silu_mul(acc[:, 0::2], acc[:, 1::2])
    dw, dx, dg = dev(torch, w), dev(torch, x), dev(torch, g)
    dy = dev(torch, y0 if epilogue == 1 else np.zeros((batch, out_n), np.uint16))
    rc = yuear_lib.lib.yuear_op_gemv(dw.data_ptr(), n, k, batch, dx.data_ptr(), k,
                                     dg.data_ptr() if norm else None, 1e-5, dy.data_ptr(), out_n,
                                     epilogue, None)
    assert rc == 0
    got = host(torch, dy)
    scale = max(np.abs(f(acc)).max(), np.abs(f(ref)).max())
    assert_close_bf16(got, ref, scale=scale, exact_frac=0.9)


@pytest.mark.parametrize("batch", [1, 2, 3, 5, 8])
def test_gemv_random_shapes_and_strides(torch, yuear_lib, oracle, batch):
    """Seeded sweep per batch size: random N, K (the MFMA form's hidden sizes
    among them), RMSNorm on or off, all three epilogues, activation rows
    padded past K and output rows padded past N; outputs against the oracle
    and every padding element of y left as it was."""
    rng = np.random.default_rng(777 + batch)
    for trial in range(6):
        k = int(rng.choice([3072, 8192, 2048, 8 * int(rng.integers(1, 1025))]))
        epilogue, norm = int(rng.integers(0, 3)), bool(rng.integers(0, 2))
        n = 2 * int(rng.integers(1, 1500)) if epilogue == 2 else int(rng.integers(1, 3000))
        out_n = n // 2 if epilogue == 2 else n
        xs, ys = k + 8 * int(rng.integers(0, 3)), out_n + int(rng.integers(0, 9))
        w = bf(rng.normal(size=(n, k)) * 0.02)
        x = bf(rng.normal(size=(batch, xs)))
        g = bf(1 + rng.normal(size=k) * 0.1)
        y0 = bf(rng.normal(size=(batch, ys)))
        xk = np.ascontiguousarray(x[:, :k])
        h = oracle.rms_norm(xk, g, 1e-5) if norm else xk
        acc = oracle.linear(h, w)
        if epilogue == 0:
            ref = acc
        elif epilogue == 1:
            ref = bf(f(y0[:, :n]) + f(acc))
        else:
            ref = oracle.silu_mul(acc[:, 0::2], acc[:, 1::2])
        dw, dx, dg, dy = dev(torch, w), dev(torch, x), dev(torch, g), dev(torch, y0)
        assert yuear_lib.lib.yuear_op_gemv(dw.data_ptr(), n, k, batch, dx.data_ptr(), xs,
                                           dg.data_ptr() if norm else None, 1e-5, dy.data_ptr(),
                                           ys, epilogue, None) == 0
        got = host(torch, dy)
        case = (trial, n, k, xs, ys, norm, epilogue)
        np.testing.assert_array_equal(got[:, out_n:], y0[:, out_n:], err_msg=str(case))
        scale = max(np.abs(f(acc)).max(), np.abs(f(ref)).max())
        assert_close_bf16(got[:, :out_n], ref, scale=scale, exact_frac=0.9)
        # overlapping rows and an empty K are refused before any launch
        for bad_xs, bad_ys, bad_k in ((k - 8, ys, k), (xs, out_n - 1, k), (xs, ys, 0)):
            assert yuear_lib.lib.yuear_op_gemv(dw.data_ptr(), n, bad_k, batch, dx.data_ptr(),
                                               bad_xs, dg.data_ptr() if norm else None, 1e-5,
                                               dy.data_ptr(), bad_ys, epilogue, None) == 1, case


def prep_qk(oracle, raw, gain, pos, theta=5e5):
    """q/k RMSNorm over each head, then RoPE at `pos` (ar.cpp:268-277)."""
    x = oracle.rms_norm(raw, gain, 1e-5) if gain is not None else raw
    return oracle.rope(x.reshape(1, -1, 128), pos, theta)[0]


@pytest.mark.parametrize("heads,kv_heads,batch_pos,splits", [
    (24, 8, [0], 64), (24, 8, [1], 64), (24, 8, [15], 64), (24, 8, [16], 64),
    (24, 8, [63], 64), (24, 8, [200], 64), (24, 8, [511], 64), (24, 8, [4095], 64),
    (24, 8, [4095], 1), (24, 8, [777], 7), (16, 8, [300], 32), (4, 2, [50], 8),
    (24, 8, [513, 1535], 32), (24, 8, [100, 1200, 7, 2047, 64, 500, 9, 1000], 32),
    (24, 8, [8191], 64),  # KV 8192: one launch of the long-context decode
    (24, 8, [24575], 64),  # the last position of the 24576-token context
    # every other accepted heads-per-kv-head ratio: G = 1 (one head per wave
    # in the prologue), 4, 6 and 8 (two and three heads per wave)
    (8, 8, [15], 64), (8, 8, [300, 4095], 32),
    (32, 8, [15], 64), (32, 8, [777], 7), (32, 8, [4095], 33),
    (48, 8, [16], 64), (48, 8, [1000, 63], 24),
    (64, 8, [15], 64), (64, 8, [2047], 16), (64, 8, [4095], 1),
])
def test_attention_decode_matches_oracle(torch, yuear_lib, oracle, heads, kv_heads, batch_pos,
                                         splits):
    rng = np.random.default_rng(sum(batch_pos) + heads + splits)
    B = len(batch_pos)
    cap = yuear_lib.kv_slots(max(batch_pos) + 9)  # V cache: whole 32-slot blocks
    qkvw = (heads + 2 * kv_heads) * 128
    qkv = bf(rng.normal(size=(B, qkvw)))
    cache_k = bf(rng.normal(size=(B, kv_heads, cap, 128)))
    cache_v = bf(rng.normal(size=(B, kv_heads, cap, 128)))
    qn, kn = bf(1 + 0.1 * rng.normal(size=128)), bf(1 + 0.1 * rng.normal(size=128))
    cos, sin = yuear_lib.rope_table(cap + 1, 128, 5e5)
    refs, kref, vref = [], [], []
    for b, pos in enumerate(batch_pos):
        q = prep_qk(oracle, qkv[b, :heads * 128].reshape(heads, 128), qn, pos)
        k = prep_qk(oracle, qkv[b, heads * 128:(heads + kv_heads) * 128].reshape(kv_heads, 128),
                    kn, pos)
        v = qkv[b, (heads + kv_heads) * 128:].reshape(kv_heads, 128)
        K, V = cache_k[b].copy(), cache_v[b].copy()
        K[:, pos], V[:, pos] = k, v
        refs.append(oracle.attention(q[None], K, V, pos)[0])
        kref.append(k)
        vref.append(v)
    args = [dev(torch, a) for a in (qkv, qn, kn, cos, sin, cache_k,
                                    yuear_lib.v_blocked(cache_v))]
    dpos = dev(torch, np.array(batch_pos, np.int32))
    out = dev(torch, np.zeros((B, heads * 128), np.uint16))
    rc = yuear_lib.lib.yuear_op_attention_decode(
        args[0].data_ptr(), args[1].data_ptr(), args[2].data_ptr(), 1e-5, args[3].data_ptr(),
        args[4].data_ptr(), args[5].data_ptr(), args[6].data_ptr(), dpos.data_ptr(), heads,
        kv_heads, cap, B, splits, out.data_ptr(), None)
    assert rc == 0
    got = host(torch, out)
    ref = np.stack(refs)
    assert_close_bf16(got, ref, exact_frac=0.8)
    gk, gv = host(torch, args[5]), yuear_lib.v_unblocked(host(torch, args[6]))
    for b, pos in enumerate(batch_pos):
        np.testing.assert_array_equal(gv[b][:, pos], vref[b])
        assert ulps_bf16(gk[b][:, pos], kref[b]).max() <= 1
        others = np.ones(cap, bool)
        others[pos] = False
        np.testing.assert_array_equal(gk[b][:, others], cache_k[b][:, others])
        np.testing.assert_array_equal(gv[b][:, others], cache_v[b][:, others])


def test_attention_decode_without_qk_norm_matches_oracle(torch, yuear_lib, oracle):
    # a model without q/k RMSNorm (null gains): RoPE only, at the last row of
    # a RoPE table sized to the position (ar.cpp:268-277 with the norms off)
    rng = np.random.default_rng(77)
    heads, kv_heads, pos = 24, 8, 1000
    cap = yuear_lib.kv_slots(pos + 1)
    qkv = bf(rng.normal(size=(1, (heads + 2 * kv_heads) * 128)))
    cache_k = bf(rng.normal(size=(1, kv_heads, cap, 128)))
    cache_v = bf(rng.normal(size=(1, kv_heads, cap, 128)))
    cos, sin = yuear_lib.rope_table(pos + 1, 128, 5e5)
    q = prep_qk(oracle, qkv[0, :heads * 128].reshape(heads, 128), None, pos)
    k = prep_qk(oracle, qkv[0, heads * 128:(heads + kv_heads) * 128].reshape(kv_heads, 128),
                None, pos)
    K, V = cache_k[0].copy(), cache_v[0].copy()
    K[:, pos], V[:, pos] = k, qkv[0, (heads + kv_heads) * 128:].reshape(kv_heads, 128)
    ref = oracle.attention(q[None], K, V, pos)
    a = [dev(torch, t) for t in (qkv, cos, sin, cache_k, yuear_lib.v_blocked(cache_v))]
    dpos = dev(torch, np.array([pos], np.int32))
    out = dev(torch, np.zeros((1, heads * 128), np.uint16))
    assert yuear_lib.lib.yuear_op_attention_decode(
        a[0].data_ptr(), None, None, 1e-5, a[1].data_ptr(), a[2].data_ptr(), a[3].data_ptr(),
        a[4].data_ptr(), dpos.data_ptr(), heads, kv_heads, cap, 1, 32, out.data_ptr(), None) == 0
    assert_close_bf16(host(torch, out), ref, exact_frac=0.8)
    assert ulps_bf16(host(torch, a[3])[0][:, pos], k).max() <= 1


def test_attention_decode_ignores_unused_slots(torch, yuear_lib):
    # vendor test_cuda_graph.py:62-79: slots beyond the position are invisible
    rng = np.random.default_rng(9)
    heads, kv, pos, cap = 24, 8, 300, 416
    qkv = bf(rng.normal(size=(1, (heads + 2 * kv) * 128)))
    k = bf(rng.normal(size=(1, kv, cap, 128)))
    v = bf(rng.normal(size=(1, kv, cap, 128)))
    cos, sin = yuear_lib.rope_table(cap, 128, 5e5)
    # slots past the position hold large values, infinities or NaNs: none may
    # reach the output (their scores are masked and their values zeroed)
    outs = []
    for poison in (None, 1000.0, np.inf, np.nan):
        kk, vv = k.copy(), v.copy()
        if poison is not None:
            kk[..., pos + 1:, :] = bf(poison)
            vv[..., pos + 1:, :] = bf(-poison)
        a = [dev(torch, t) for t in (qkv, cos, sin, kk, yuear_lib.v_blocked(vv))]
        dpos = dev(torch, np.array([pos], np.int32))
        out = dev(torch, np.zeros((1, heads * 128), np.uint16))
        assert yuear_lib.lib.yuear_op_attention_decode(
            a[0].data_ptr(), None, None, 1e-5, a[1].data_ptr(), a[2].data_ptr(), a[3].data_ptr(),
            a[4].data_ptr(), dpos.data_ptr(), heads, kv, cap, 1, 16, out.data_ptr(), None) == 0
        outs.append(host(torch, out))
    for o in outs[1:]:
        np.testing.assert_array_equal(outs[0], o)


@pytest.mark.parametrize("m,n,k,residual", [
    (1, 256, 256, 0), (7, 1024, 3072, 0), (128, 5120, 3072, 0), (129, 3072, 3072, 1),
    (300, 1024, 8192, 1), (1000, 384, 512, 0),
])
def test_gemm_matches_oracle(torch, yuear_lib, oracle, m, n, k, residual):
    rng = np.random.default_rng(m * 7 + n)
    a = bf(rng.normal(size=(m, k)))
    w = bf(rng.normal(size=(n, k)) * 0.02)
    c0 = bf(rng.normal(size=(m, n)))
    acc = oracle.linear(a, w)
    ref = bf(f(c0) + f(acc)) if residual else acc
    da, dw = dev(torch, a), dev(torch, w)
    dc = dev(torch, c0 if residual else np.zeros((m, n), np.uint16))
    assert yuear_lib.lib.yuear_op_gemm(da.data_ptr(), k, dw.data_ptr(), m, n, k, dc.data_ptr(),
                                       n, residual, None) == 0
    scale = max(np.abs(f(acc)).max(), np.abs(f(ref)).max())
    assert_close_bf16(host(torch, dc), ref, scale=scale, exact_frac=0.9)


@pytest.mark.parametrize("m,n,k,residual", [
    (3000, 5120, 3072, 0), (3000, 3072, 3072, 1), (3000, 16384, 3072, 0), (3000, 3072, 8192, 1),
    (4096, 16384, 3072, 0), (2049, 3072, 8192, 1),
])
def test_gemm_prefill_shapes(torch, yuear_lib, oracle, m, n, k, residual):
    """The four projections of a prefill (QKV, output, gate/up, down) at
    3000, 4096 and 2049 tokens (large enough for the 256 x 256 tile on a
    256-CU part, and a ragged last tile row): 96 rows, among them the first
    and last of every 256-row tile, against the oracle."""
    rng = np.random.default_rng(m + n + k)
    a = bf(rng.normal(size=(m, k)))
    w = bf(rng.normal(size=(n, k)) * 0.02)
    c0 = bf(rng.normal(size=(m, n))) if residual else np.zeros((m, n), np.uint16)
    da, dw, dc = dev(torch, a), dev(torch, w), dev(torch, c0)
    assert yuear_lib.lib.yuear_op_gemm(da.data_ptr(), k, dw.data_ptr(), m, n, k, dc.data_ptr(),
                                       n, residual, None) == 0
    got = host(torch, dc)
    edges = [r for t in range(0, m, 256) for r in (t, min(t + 255, m - 1))]
    rows = np.unique(np.concatenate([edges, rng.integers(0, m, size=96 - len(set(edges)))]))
    acc = oracle.linear(a[rows], w)
    ref = bf(f(c0[rows]) + f(acc)) if residual else acc
    scale = max(np.abs(f(acc)).max(), np.abs(f(ref)).max())
    assert_close_bf16(got[rows], ref, scale=scale, exact_frac=0.9)


@pytest.mark.parametrize("shape", range(6))
@pytest.mark.parametrize("m,n,k", [(300, 1000, 512), (3000, 16384, 3072), (5, 36, 64)])
def test_gemm_swiglu_epilogue(torch, yuear_lib, oracle, shape, m, n, k):
    """The SwiGLU form (residual = 2) on interleaved gate/up rows against the
    oracle's linear + silu_mul (ar.cpp:36-51), every tile shape; at the
    3B gate/up shape a sample of rows."""
    rng = np.random.default_rng(m + shape)
    a = bf(rng.normal(size=(m, k)))
    w = bf(rng.normal(size=(n, k)) * 0.03)
    da, dw = dev(torch, a), dev(torch, w)
    dc = dev(torch, np.zeros((m, n // 2), np.uint16))
    assert yuear_lib.lib.yuear_op_gemm_tile(da.data_ptr(), k, dw.data_ptr(), m, n, k,
                                            dc.data_ptr(), n // 2, 2, shape, None) == 0
    got = host(torch, dc)
    rows = np.arange(m) if m <= 300 else np.unique(np.r_[0, m - 1, rng.integers(0, m, 40)])
    acc = oracle.linear(a[rows], w)
    ref = oracle.silu_mul(acc[:, 0::2], acc[:, 1::2])
    assert_close_bf16(got[rows], ref, exact_frac=0.9)
    # odd n is rejected for the SwiGLU form
    assert yuear_lib.lib.yuear_op_gemm_tile(da.data_ptr(), k, dw.data_ptr(), m, n - 1, k,
                                            dc.data_ptr(), n // 2, 2, shape, None) == 1


def test_gemm_swiglu_every_gate_value(torch, yuear_lib, oracle):
    """The GEMM's SwiGLU epilogue depends on the bf16 gate value alone (up
    rounded apart), so all 65536 of them are checked (gate column i = bf16
    bits i, up = 1, A = e_0): bit for bit against the decode GEMV's SwiGLU
    (gemv_core.h) on every tile shape and through split-K's reduce kernel,
    and against the oracle's silu_mul (ar.cpp:36-51) within the bf16 bound
    for the finite ones."""
    k, pairs = 128, 65536
    a = np.zeros((1, k), np.uint16)
    a[0, 0] = 0x3F80  # 1.0
    w = np.zeros((2 * pairs, k), np.uint16)
    w[0::2, 0] = np.arange(pairs, dtype=np.uint32).astype(np.uint16)
    w[1::2, 0] = 0x3F80
    da, dw = dev(torch, a), dev(torch, w)
    dy = dev(torch, np.zeros((1, pairs), np.uint16))
    assert yuear_lib.lib.yuear_op_gemv(dw.data_ptr(), 2 * pairs, k, 1, da.data_ptr(), k, None,
                                       1e-5, dy.data_ptr(), pairs, 2, None) == 0
    want = host(torch, dy)[0]
    runs = [(shape, 1) for shape in range(6)] + [(4, 2)]
    for shape, splits in runs:
        dc = dev(torch, np.zeros((1, pairs), np.uint16))
        assert yuear_lib.lib.yuear_op_gemm_split(da.data_ptr(), k, dw.data_ptr(), 1, 2 * pairs, k,
                                                 dc.data_ptr(), pairs, 2, shape, splits,
                                                 None) == 0
        got = host(torch, dc)[0]
        bad = np.flatnonzero(got != want)
        print(f"shape {shape} splits {splits}: {bad.size} of {pairs} differ from the GEMV",
              [(hex(int(i)), hex(int(got[i])), hex(int(want[i]))) for i in bad[:6]], flush=True)
        assert bad.size == 0
    gate = f(w[0::2, 0])
    finite = np.isfinite(gate) & np.isfinite(f(want))
    ref = oracle.silu_mul(w[0::2, 0][None, :], w[1::2, 0][None, :])[0]
    assert_close_bf16(want[finite], ref[finite], scale=2.0 ** -100, exact_frac=0.99)


@pytest.mark.parametrize("shape", range(6))
@pytest.mark.parametrize("m,n,k,residual", [(300, 1000, 512, 0), (517, 776, 192, 1), (1, 200, 64, 1)])
def test_gemm_every_tile_shape(torch, yuear_lib, oracle, shape, m, n, k, residual):
    """Each of the six tile shapes, forced, on ragged sizes (M and N not
    multiples of any tile, N not a multiple of 8, single-row M)."""
    rng = np.random.default_rng(m + n + shape)
    a = bf(rng.normal(size=(m, k)))
    w = bf(rng.normal(size=(n, k)) * 0.05)
    c0 = bf(rng.normal(size=(m, n))) if residual else np.zeros((m, n), np.uint16)
    acc = oracle.linear(a, w)
    ref = bf(f(c0) + f(acc)) if residual else acc
    da, dw, dc = dev(torch, a), dev(torch, w), dev(torch, c0)
    assert yuear_lib.lib.yuear_op_gemm_tile(da.data_ptr(), k, dw.data_ptr(), m, n, k,
                                            dc.data_ptr(), n, residual, shape, None) == 0
    scale = max(np.abs(f(acc)).max(), np.abs(f(ref)).max())
    assert_close_bf16(host(torch, dc), ref, scale=scale, exact_frac=0.9)
    assert yuear_lib.lib.yuear_op_gemm_tile(da.data_ptr(), k, dw.data_ptr(), m, n, k,
                                            dc.data_ptr(), n, residual, 6, None) == 1


@pytest.mark.parametrize("shape", range(6))
def test_gemm_random_shapes_and_strides(torch, yuear_lib, oracle, shape):
    """Seeded sweep per tile shape: ragged M, N and K, A rows padded past K
    (lda > k, the padding filled with other values), C rows padded past the
    output (ldc > n, odd strides included) and all three epilogues; outputs
    against the oracle, and every padding element of C left as it was."""
    rng = np.random.default_rng(4242 + shape)
    for trial in range(5):
        m, k = int(rng.integers(1, 600)), 64 * int(rng.integers(1, 13))
        residual = int(rng.integers(0, 3))
        n = 2 * int(rng.integers(1, 450)) if residual == 2 else int(rng.integers(1, 900))
        out_n = n // 2 if residual == 2 else n
        lda, ldc = k + 8 * int(rng.integers(0, 3)), out_n + int(rng.integers(0, 6))
        a = bf(rng.normal(size=(m, lda)))
        w = bf(rng.normal(size=(n, k)) * 0.05)
        c0 = bf(rng.normal(size=(m, ldc)) * (1.0 if residual == 1 else 7.0))
        da, dw, dc = dev(torch, a), dev(torch, w), dev(torch, c0)
        assert yuear_lib.lib.yuear_op_gemm_tile(da.data_ptr(), lda, dw.data_ptr(), m, n, k,
                                                dc.data_ptr(), ldc, residual, shape, None) == 0
        got = host(torch, dc)
        acc = oracle.linear(np.ascontiguousarray(a[:, :k]), w)
        if residual == 2:
            ref = oracle.silu_mul(acc[:, 0::2], acc[:, 1::2])
        elif residual == 1:
            ref = bf(f(c0[:, :n]) + f(acc))
        else:
            ref = acc
        case = (trial, m, n, k, lda, ldc, residual)
        np.testing.assert_array_equal(got[:, out_n:], c0[:, out_n:], err_msg=str(case))
        scale = max(np.abs(f(acc)).max(), np.abs(f(ref)).max()) if residual != 2 else None
        assert_close_bf16(got[:, :out_n], ref, scale=scale, exact_frac=0.9)


@pytest.mark.parametrize("m,n,k,residual,splits", [
    (300, 1000, 512, 0, 2), (517, 776, 1024, 1, 4), (129, 200, 3072, 2, 6),
    (64, 3072, 8192, 1, 8), (1, 200, 1024, 0, 16)])
def test_gemm_split_k_matches_oracle(torch, yuear_lib, oracle, m, n, k, residual, splits):
    """The split-K form (each split's K range summed into fp32 partials, the
    splits added in split order before the epilogue) on every tile shape:
    against the oracle, identical bits on a second launch, and a split count
    that does not divide K's 64-wide steps refused."""
    rng = np.random.default_rng(m + n + k + splits)
    a = bf(rng.normal(size=(m, k)))
    w = bf(rng.normal(size=(n, k)) * 0.05)
    out_n = n // 2 if residual == 2 else n
    c0 = bf(rng.normal(size=(m, out_n))) if residual == 1 else np.zeros((m, out_n), np.uint16)
    acc = oracle.linear(a, w)
    if residual == 2:
        ref, scale = oracle.silu_mul(acc[:, 0::2], acc[:, 1::2]), None
    else:
        ref = bf(f(c0) + f(acc)) if residual else acc
        scale = max(np.abs(f(acc)).max(), np.abs(f(ref)).max())
    da, dw = dev(torch, a), dev(torch, w)
    for shape in range(6):
        outs = []
        for _ in range(2):
            dc = dev(torch, c0)
            assert yuear_lib.lib.yuear_op_gemm_split(da.data_ptr(), k, dw.data_ptr(), m, n, k,
                                                     dc.data_ptr(), out_n, residual, shape,
                                                     splits, None) == 0
            outs.append(host(torch, dc))
        np.testing.assert_array_equal(outs[0], outs[1], err_msg=f"shape {shape}")
        assert_close_bf16(outs[0], ref, scale=scale, exact_frac=0.9)
    bad = next(z for z in range(2, 17) if (k // 64) % z)
    assert yuear_lib.lib.yuear_op_gemm_split(da.data_ptr(), k, dw.data_ptr(), m, n, k,
                                             dev(torch, c0).data_ptr(), out_n, residual, 0, bad,
                                             None) == 1
    # refused before any workspace is sized: a workspace beyond size_t, and K
    # that is no whole number of 64-wide steps
    huge = 1 << 30
    assert yuear_lib.lib.yuear_op_gemm_split(da.data_ptr(), k, dw.data_ptr(), huge, huge, k,
                                             dev(torch, c0).data_ptr(), huge, 0, 0, 2,
                                             None) == 1
    assert yuear_lib.lib.yuear_op_gemm_split(da.data_ptr(), k, dw.data_ptr(), m, n, k - 32,
                                             dev(torch, c0).data_ptr(), out_n, residual, 0, 2,
                                             None) == 1


@pytest.mark.parametrize("m,n,k", [(7, 1024, 3072), (3000, 3072, 8192), (700, 5120, 3072)])
def test_gemm_split_k_is_deterministic(torch, yuear_lib, m, n, k):
    """Every output sums its K products in the same order on each launch (no
    atomics; yuear_op_gemm has no workspace, so K is never split), so
    repeated launches of narrow, wide and deep shapes give identical bits."""
    rng = np.random.default_rng(m + 3 * n)
    a = dev(torch, bf(rng.normal(size=(m, k))))
    w = dev(torch, bf(rng.normal(size=(n, k)) * 0.02))
    outs = []
    for _ in range(3):
        c = dev(torch, np.zeros((m, n), np.uint16))
        assert yuear_lib.lib.yuear_op_gemm(a.data_ptr(), k, w.data_ptr(), m, n, k, c.data_ptr(),
                                           n, 0, None) == 0
        outs.append(host(torch, c))
    for o in outs[1:]:
        np.testing.assert_array_equal(outs[0], o)


def test_op_scratch_is_per_stream(torch, yuear_lib):
    """Residual GEMMs and decode attentions issued on two streams at once
    equal the same calls made one at a time: the op-level scratch (split
    partials and counters) is never shared between streams, and the GEMM
    keeps nothing between calls."""
    rng = np.random.default_rng(31)
    m, n, k = 300, 3072, 3072
    heads, kv, pos, cap = 24, 8, 700, 736
    cos, sin = yuear_lib.rope_table(cap, 128, 5e5)
    dcos, dsin = dev(torch, cos), dev(torch, sin)
    dpos = dev(torch, np.array([pos], np.int32))
    jobs = []
    for j in range(2):
        a = dev(torch, bf(rng.normal(size=(m, k))))
        w = dev(torch, bf(rng.normal(size=(n, k)) * 0.02))
        c0 = dev(torch, bf(rng.normal(size=(m, n))))
        qkv = dev(torch, bf(rng.normal(size=(1, (heads + 2 * kv) * 128))))
        kc = dev(torch, bf(rng.normal(size=(1, kv, cap, 128))))
        vc = dev(torch, yuear_lib.v_blocked(bf(rng.normal(size=(1, kv, cap, 128)))))
        jobs.append((a, w, c0, qkv, kc, vc))
    lib = yuear_lib.lib

    def run(job, c, out, stream):
        a, w, _, qkv, kc, vc = job
        assert lib.yuear_op_gemm(a.data_ptr(), k, w.data_ptr(), m, n, k, c.data_ptr(), n, 1,
                                 stream) == 0
        assert lib.yuear_op_attention_decode(
            qkv.data_ptr(), None, None, 1e-5, dcos.data_ptr(), dsin.data_ptr(), kc.data_ptr(),
            vc.data_ptr(), dpos.data_ptr(), heads, kv, cap, 1, 16, out.data_ptr(), stream) == 0

    # serial reference on one stream (the KV append writes the same slot
    # again in the concurrent pass, with the same values)
    ref = []
    for job in jobs:
        c, out = job[2].clone(), torch.zeros((1, heads * 128), dtype=torch.int16, device="cuda")
        run(job, c, out, None)
        torch.cuda.synchronize()
        ref.append((host(torch, c), host(torch, out)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        got = []
        for job, st in zip(jobs, streams):
            c, out = job[2].clone(), torch.zeros((1, heads * 128), dtype=torch.int16,
                                                 device="cuda")
            torch.cuda.synchronize()
            got.append((c, out, st))
        for (c, out, st), job in zip(got, jobs):
            run(job, c, out, st.cuda_stream)
        torch.cuda.synchronize()
        for (c, out, _), (rc, ro) in zip(got, ref):
            np.testing.assert_array_equal(host(torch, c), rc)
            np.testing.assert_array_equal(host(torch, out), ro)


@pytest.mark.parametrize("T,pos0,heads,kv_heads", [(7, 0, 4, 2), (64, 0, 24, 8),
                                                   (65, 10, 24, 8), (200, 333, 16, 8),
                                                   # 24 x 33 = 792 workgroups of 64 queries:
                                                   # the LDS-shared tile, ragged last tile
                                                   (2100, 40, 24, 8),
                                                   # the 3000-token prefill, one pass and
                                                   # its last chunk after 2048 cached keys
                                                   (3000, 0, 24, 8), (952, 2048, 24, 8),
                                                   # 384 workgroups, the fewest that take the
                                                   # 64-query tile (ragged last tile after 100)
                                                   (1024, 0, 24, 8), (1000, 100, 24, 8),
                                                   # the last 100 queries of the 24576-token
                                                   # context
                                                   (100, 24476, 24, 8)])
def test_attention_prefill_matches_oracle(torch, yuear_lib, oracle, T, pos0, heads, kv_heads):
    rng = np.random.default_rng(T + pos0)
    cap = yuear_lib.kv_slots(pos0 + T + 3)
    q = bf(rng.normal(size=(T, heads, 128)))
    kc = bf(rng.normal(size=(kv_heads, cap, 128)))
    vc = bf(rng.normal(size=(kv_heads, cap, 128)))
    ref = oracle.attention(q, kc, vc, pos0)
    a = [dev(torch, t) for t in (q, kc, yuear_lib.v_blocked(vc))]
    out = dev(torch, np.zeros((T, heads * 128), np.uint16))
    assert yuear_lib.lib.yuear_op_attention_prefill(a[0].data_ptr(), a[1].data_ptr(),
                                                    a[2].data_ptr(), T, pos0, heads, kv_heads,
                                                    cap, out.data_ptr(), None) == 0
    assert_close_bf16(host(torch, out), ref, exact_frac=0.8)
    # a negative start, a range past the capacity and a head count below the
    # kv heads are refused before any launch
    for t_, p0, hq in ((T, -1, heads), (T, cap - T + 1, heads), (T, pos0, 0)):
        assert yuear_lib.lib.yuear_op_attention_prefill(
            a[0].data_ptr(), a[1].data_ptr(), a[2].data_ptr(), t_, p0, hq, kv_heads, cap,
            out.data_ptr(), None) == 1, (t_, p0, hq)
