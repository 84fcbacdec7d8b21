"""GPU parity: gated-GQA drop-in ops through the C ABI against the oracle.

RMSNorm and RoPE have no libm-dependent step on the device (sqrt and
divide are correctly rounded; RoPE's cos/sin codes come from the host
table) and must be bit-identical. Eager GQA and the output gate evaluate
expf correctly rounded on the device and are held to 1 bf16 ulp and 2e-3
relative (tests/numerics.py); decode must equal the last row of a full
recompute bitwise, as in the reference (c/attn.h:49-52).
"""
import numpy as np
import pytest

import synth
from numerics import assert_bf16_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N", [256, 1023, 2048])
def test_rmsnorm_bitwise(hip, orc, rng, N):
    x = synth.normal_bf16(rng, (N,), 2.0)
    w = synth.normal_bf16(rng, (N,), 0.1)
    assert np.array_equal(hip.attn_rmsnorm(x, w), orc.attn_rmsnorm(x, w))
    z = np.zeros(N, np.uint16)
    assert (hip.attn_rmsnorm(z, w) == 0).all()


@pytest.mark.parametrize("pos", [0.0, 1.0, 7.0, 1000.0, 32767.0, 131071.0, 262143.0])
def test_rope_bitwise(hip, orc, rng, pos):
    x = synth.normal_bf16(rng, (256,))
    y = hip.attn_rope(x, 64, pos)
    assert np.array_equal(y, orc.attn_rope(x, 64, pos))
    if pos == 0.0:
        assert np.array_equal(y, x)


@pytest.mark.parametrize("Tq,Tk,H,Hkv,D", [(6, 6, 4, 2, 64), (7, 7, 3, 1, 65), (1, 300, 16, 2, 256),
                                           (5, 517, 16, 2, 256)])
def test_gqa(hip, orc, rng, Tq, Tk, H, Hkv, D):
    q = synth.normal_bf16(rng, (Tq * H * D,))
    kc = synth.normal_bf16(rng, (Tk * Hkv * D,))
    vc = synth.normal_bf16(rng, (Tk * Hkv * D,), 1.2)
    scale = np.float32(1.0 / np.sqrt(D))
    o = hip.attn_gqa(q, kc, vc, Tq, Tk, H, Hkv, D, scale)
    st = assert_bf16_close(o, orc.attn_gqa(q, kc, vc, Tq, Tk, H, Hkv, D, scale), what="gqa")
    print(st)
    od = hip.attn_gqa_decode(q[(Tq - 1) * H * D:].copy(), kc, vc, Tk, H, Hkv, D, scale)
    assert np.array_equal(od, o[(Tq - 1) * H * D:])


def test_outgate(hip, orc, rng):
    o = synth.normal_bf16(rng, (4099,), 1.5)
    g = synth.normal_bf16(rng, (4099,), 4.0)
    assert_bf16_close(hip.attn_outgate(o, g), orc.attn_outgate(o, g), what="outgate")
    gc = synth.bf16_bits(np.array([0.0, 20.0], np.float32))
    oc = o[:2].copy()
    y = hip.attn_outgate(oc, gc)
    assert y[1] == oc[1]
    assert y[0] == synth.bf16_bits(np.array([synth.bf16_f32(oc[:1])[0] * np.float32(0.5)], np.float32))[0]
