"""The host quantizer behind the RANDOM weight source's "8bit" / "4bit"
linears (yuear_quantize_affine; the conversion step of
native/src/conversion.cpp:470-532, mx::quantize(w, 64, bits, "affine")), on
the CPU. Its agreement with MLX's own quantizer is parity unpinned (MLX is
absent); what is checked is what the affine format fixes: codes in range,
every dequantized weight within half a step of the original, the edge of
larger magnitude reproduced exactly, and the packing order read back through
the byte view of the words.
"""
import numpy as np
import pytest

from quant_util import bf, dequantize_f64, unpack_bytes


def f(bits):
    import cpu_ref
    return cpu_ref.bf16_to_f32(bits)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_affine_bounds_and_edges(yuear_lib, bits):
    rng = np.random.default_rng(bits)
    w = bf(rng.normal(size=(33, 512)) * 0.02)
    w[3, :64] = bf(np.full(64, 0.25))          # constant group
    w[4, 64:128] = 0                            # zero group
    codes, scales, biases = yuear_lib.quantize_affine(w, bits)
    assert codes.shape == (33, 512 * bits // 32) and scales.shape == biases.shape == (33, 8)
    q = unpack_bytes(codes, bits)
    assert q.min() >= 0 and q.max() <= (1 << bits) - 1
    deq = dequantize_f64(q, scales, biases)
    wf = f(w).astype(np.float64)
    step = np.repeat(np.abs(f(scales)).astype(np.float64), 64, axis=1)
    # codes strictly inside the range round to the nearest step; the end
    # codes may be clipped, since the scale is refined to edge / round(edge /
    # scale) (zero falls on a code), which can move the far end past the last
    # code by up to about one step
    err = np.abs(deq - wf) / step
    inner = (q > 0) & (q < (1 << bits) - 1)
    assert err[inner].max() <= 0.5 + 1e-6
    assert err.max() <= 1.5
    groups = wf.reshape(33, 8, 64)
    edge = np.where(np.abs(groups.min(-1)) > np.abs(groups.max(-1)), groups.min(-1),
                    groups.max(-1))
    deqg = deq.reshape(33, 8, 64)
    hit = np.isclose(deqg, edge[..., None], rtol=0, atol=0).any(-1)
    assert hit.all()
    assert np.all(deq[3, :64] == 0.25) and np.all(deq[4, 64:128] == 0)
