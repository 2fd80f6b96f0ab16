"""Acoustic-model attention on the GPU (yuear_nar_attention, the drop-in for
nar_attention() and its Metal kernel lyra_nar_precise_attention,
nar_attention.cpp:63-270) against the oracle's restatement, at the
conditioning and acoustic-chunk shapes of the 3B / YuE2 layers and at the
edges (one query, one key, key counts off the 32-key blocks, causal), plus
the reference's ValueError checks (nar_attention.cpp:227-243)."""
import numpy as np
import pytest

from conftest import assert_close_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    t.cuda.init()
    return t


def bf(x):
    import cpu_ref
    return cpu_ref.f32_to_bf16(np.asarray(x, dtype=np.float32))


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)


def host(torch, t):
    torch.cuda.synchronize()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,causal", [
    (1, 16, 8, 130, 700, False),   # YuE2 heads: acoustic chunk over cached AR keys + its own
    (1, 24, 8, 300, 1100, False),  # 3B heads
    (2, 4, 2, 9, 65, False),       # batch 2, short chunk, keys off the 32-key blocks
    (1, 4, 2, 1, 33, False),       # one query
    (1, 4, 4, 40, 1, False),       # one key
    (1, 16, 8, 257, 257, True),    # causal conditioning prefill
    (2, 6, 3, 64, 64, True),
    # >= 768 workgroups of 64 queries: the LDS-shared 64-query tile (ragged last tiles)
    (2, 24, 8, 1000, 1100, False),
    (1, 24, 8, 2050, 2050, True),
    (32, 24, 8, 64, 1, False),     # 768 workgroups of 64 queries over one key
    (16, 24, 8, 130, 130, True),   # 1152 workgroups, causal, 2-query last tiles
    # keys split over workgroups (fewer than 768 workgroups of 64 queries)
    (1, 16, 8, 64, 2570, False),   # 81 key blocks: 9 splits of 9, none empty
    (1, 24, 8, 512, 3512, False),  # the benchmarked acoustic chunk over conditioning keys
    (1, 16, 8, 4, 3100, False),    # 4 queries in one 64-query tile, 12 splits
    (2, 16, 8, 100, 1500, False),  # batch 2, 5 splits, ragged last query tile
])
def test_nar_attention_matches_oracle(torch, yuear_lib, oracle, B, Hq, Hkv, Lq, Lk, causal):
    print(f"[nar] B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} causal={causal}", flush=True)
    rng = np.random.default_rng(Lq * 7 + Lk)
    q = bf(rng.normal(size=(B, Hq, Lq, 128)))
    k = bf(rng.normal(size=(B, Hkv, Lk, 128)))
    v = bf(rng.normal(size=(B, Hkv, Lk, 128)))
    ref = oracle.nar_attention(q, k, v, causal)
    got = yuear_lib.nar_attention(dev(torch, q), dev(torch, k), dev(torch, v), causal)
    assert_close_bf16(host(torch, got), ref, exact_frac=0.8)


def test_nar_attention_zero_pads_the_last_key_block(torch, yuear_lib, oracle):
    # 50 keys leave 14 padding slots in the last 32-key block of the
    # workspace: a workspace full of NaN must not reach the output
    rng = np.random.default_rng(1)
    q = bf(rng.normal(size=(1, 4, 20, 128)))
    k = bf(rng.normal(size=(1, 2, 50, 128)))
    v = bf(rng.normal(size=(1, 2, 50, 128)))
    nbytes = yuear_lib.lib.yuear_nar_attention_workspace_bytes(1, 2, 50)
    assert nbytes == 2 * 64 * 128 * 2
    ws = dev(torch, np.full(nbytes // 2, 0x7FC0, np.uint16))
    got = host(torch, yuear_lib.nar_attention(dev(torch, q), dev(torch, k), dev(torch, v),
                                              workspace=ws))
    import cpu_ref
    assert not np.isnan(cpu_ref.bf16_to_f32(got)).any()
    assert_close_bf16(got, oracle.nar_attention(q, k, v), exact_frac=0.8)


def test_nar_attention_errors(torch, yuear_lib):
    x = dev(torch, np.zeros((1, 4, 8, 128), np.uint16))
    w = torch.empty(1 << 16, dtype=torch.uint8, device="cuda")
    lib = yuear_lib.lib
    import ctypes as C

    def call(heads, kv_heads, q_len, kv_len, head_dim=128, causal=0, chunk=64):
        err = C.c_void_p()
        st = lib.yuear_nar_attention(x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, heads,
                                     kv_heads, q_len, kv_len, head_dim, causal, chunk,
                                     w.data_ptr(), x.data_ptr(), None, C.byref(err))
        msg = C.string_at(err.value).decode() if err.value else ""
        if err.value:
            lib.yuear_string_free(err)
        return st, msg

    st, msg = call(4, 3, 8, 8)
    assert st == 2 and "Invalid grouped-query head count" in msg
    assert "nonempty" in call(4, 2, 0, 8)[1]
    assert "equal query and key lengths" in call(4, 2, 8, 4, causal=1)[1]
    assert "query_chunk_size" in call(4, 2, 8, 8, chunk=0)[1]
    assert "head_dim 128" in call(4, 2, 8, 8, head_dim=64)[1]
    assert call(4, 2, 8, 8)[0] == 0


def test_nar_condition_is_the_prefill_cache(torch, yuear_lib, oracle):
    """CachedNAR's conditioning prefill (nar.cpp:139-190): the keys and values
    of the visible prefix equal the engine's prefill cache bit for bit and the
    oracle's within the prefill tolerance."""
    from conftest import TINY
    w = yuear_lib.random_weights(TINY, seed=8, norm_std=0.1)
    engine = yuear_lib.Engine(TINY, w)
    model = oracle.Model(TINY, w)
    ids = [5, 9, 14, 200, 33, 1, 511, 256, 3, 77, 12, 40, 41, 42]
    for visible_end in (0, 9, 100):
        print(f"[nar condition] visible_end={visible_end}", flush=True)
        k, v = engine.nar_condition(ids, visible_end)
        vis = min(visible_end, len(ids)) if visible_end else len(ids)
        assert tuple(k.shape) == (TINY["num_hidden_layers"], TINY["num_key_value_heads"], vis, 128)
        s = engine.session(1, 32)
        s.prefill(0, ids)
        cache = model.cache(32)
        model.hidden(ids, cache)
        kh, vh = host(torch, k), host(torch, v)
        for layer in range(TINY["num_hidden_layers"]):
            ks, vs = s.read_kv(layer, 0, len(ids))
            np.testing.assert_array_equal(kh[layer], ks[:, :vis])
            np.testing.assert_array_equal(vh[layer], vs[:, :vis])
            assert_close_bf16(kh[layer], cache.keys(layer)[:, :vis], exact_frac=0.8)
            assert_close_bf16(vh[layer], cache.values(layer)[:, :vis], exact_frac=0.8)
        s.close()
    with pytest.raises(ValueError, match="outside the model vocabulary"):
        engine.nar_condition([1, 2, 512])
    with pytest.raises(ValueError, match="nonnegative"):
        engine.nar_condition([1, 2], -1)
    engine.close()
    q = yuear_lib.Engine(TINY, seed=3, bits=4)
    with pytest.raises(ValueError, match="quantized AR cannot condition NAR"):
        q.nar_condition([1, 2, 3])
    q.close()


def test_nar_attention_graph_survives_a_larger_call(torch, yuear_lib):
    """The split partials come from a pool per (device, stream). A graph
    captured on a stream keeps the pool buffer it was captured with: a later
    call on that stream that needs a larger buffer allocates a new one and
    keeps the old one alive, so replays of the graph stay correct."""
    rng = np.random.default_rng(21)

    def inputs(lk):
        return (dev(torch, bf(rng.normal(size=(1, 16, 64, 128)))),
                dev(torch, bf(rng.normal(size=(1, 8, lk, 128)))),
                dev(torch, bf(rng.normal(size=(1, 8, lk, 128)))))

    small, large = inputs(600), inputs(2570)  # 2 and 9 key splits
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        ws = torch.empty(yuear_lib.lib.yuear_nar_attention_workspace_bytes(1, 8, 2570) // 2,
                         dtype=torch.bfloat16, device="cuda")
        want = yuear_lib.nar_attention(*small, workspace=ws, stream=s.cuda_stream)
        want = host(torch, want)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = yuear_lib.nar_attention(*small, workspace=ws, stream=s.cuda_stream)
        big = host(torch, yuear_lib.nar_attention(*large, workspace=ws, stream=s.cuda_stream))
        for replay in range(3):
            out.zero_()
            g.replay()
            np.testing.assert_array_equal(host(torch, out), want, err_msg=f"replay {replay}")
    again = host(torch, yuear_lib.nar_attention(*large, workspace=ws, stream=s.cuda_stream))
    np.testing.assert_array_equal(again, big)
