"""CPU checks of the attention tolerance helper (tests/attn_util.py): the
rounding-flip allowance recognises bf16 midpoints, stays a small fraction
of the term scale, and does not absorb real mistakes (an attention that
drops its last key, or reads the key before it, fails the bar)."""
import numpy as np
import pytest

import synth
from attn_util import _midpoint_dist, attn_esc_rows
from numerics import assert_bf16_esc


def test_midpoints():
    d, ulp = _midpoint_dist(np.array([1.0 + 2.0 ** -8, 1.0, 3.0, -24.0625]))
    assert d[0] == 0.0 and ulp[0] == 2.0 ** -7
    assert d[1] == 2.0 ** -8                       # a code is half an ulp from a midpoint
    assert ulp[2] == 2.0 ** -6 and ulp[3] == 2.0 ** -3
    assert d[3] == 0.0                             # 24.0625 = 24 + ulp/2


def _case(orc, seed, n_keys=96):
    rng = np.random.default_rng(seed)
    nh, nkv, d = 16, 2, 256
    q = synth.normal_bf16(rng, (1, nh * d))
    K = synth.normal_bf16(rng, (n_keys, nkv, d))
    V = synth.normal_bf16(rng, (n_keys, nkv, d))
    return q, K, V, nh, nkv, d


def test_allowance_is_small(orc):
    q, K, V, nh, nkv, d = _case(orc, 1)
    pos = np.array([95])
    e0 = attn_esc_rows(q, K, V, pos, nh, nkv, d, flips=False)
    e1 = attn_esc_rows(q, K, V, pos, nh, nkv, d)
    assert np.all(e1 >= e0)
    assert np.median(e1 / e0) < 2.0                # about 1e-3 of esc on top of 2e-3


@pytest.mark.parametrize("seed", [2, 3, 4])
def test_mistakes_fail(orc, seed):
    q, K, V, nh, nkv, d = _case(orc, seed)
    sc = np.float32(1.0 / 16.0)
    good = orc.attn_gqa(q, K, V, 1, 96, nh, nkv, d, sc)
    esc = attn_esc_rows(q, K, V, np.array([95]), nh, nkv, d)
    assert_bf16_esc(good, good, esc, ulps=2)
    dropped = orc.attn_gqa(q, np.ascontiguousarray(K[:95]), np.ascontiguousarray(V[:95]), 1, 95,
                           nh, nkv, d, sc)
    with pytest.raises(AssertionError):
        assert_bf16_esc(dropped, good, esc, ulps=2)
    K2 = K.copy()
    K2[95] = K[94]                                 # off-by-one key row
    shifted = orc.attn_gqa(q, K2, V, 1, 96, nh, nkv, d, sc)
    with pytest.raises(AssertionError):
        assert_bf16_esc(shifted, good, esc, ulps=2)
