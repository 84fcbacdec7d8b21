"""Pin the oracle restatement BITWISE against the reference's own scalar
anchors, compiled from /root/reference/c into oracle/_ref (oracle/Makefile).

Each op is run on identical seeded inputs through both libraries; every
output byte and every in/out state byte must match. Shapes include odd
sizes (tails) and the model's real dims. The mixer drivers add the
wiring of c/layer.h (repeat-interleave, rnd before onorm, append before
attention, per-sequence state) on multi-sequence, multi-token batches.
"""
import numpy as np
import pytest

import synth
from synth import bf16_bits


def _f32(rng, n, s=1.0):
    return (rng.standard_normal(n, dtype=np.float32) * np.float32(s))


@pytest.mark.parametrize("C,T", [(37, 9), (8192, 3)])
def test_conv1d_bitwise(orc, ref, rng, C, T):
    x = synth.normal_bf16(rng, (T, C), 1.5)
    w = synth.normal_bf16(rng, (C, 4), 0.7)
    st0 = synth.normal_bf16(rng, (C * 3,))
    s1, s2 = st0.copy(), st0.copy()
    assert np.array_equal(orc.gdn_conv1d(x, w, s1), ref.gdn_conv1d(x, w, s2))
    assert np.array_equal(s1, s2)
    s3 = st0.copy()
    step = np.stack([orc.gdn_conv1d_step(x[t].copy(), w, s3) for t in range(T)])
    assert np.array_equal(step, orc.gdn_conv1d(x, w, st0.copy()))
    assert np.array_equal(s3, s1)


def test_decay_beta_bitwise(orc, ref, rng):
    H = 4099
    a = synth.normal_bf16(rng, (H,), 3.0)
    b = synth.normal_bf16(rng, (H,), 6.0)
    A = rng.uniform(-1, 2.7, H).astype(np.float32)
    dt = _f32(rng, H, 4.0)
    dt[:5] = [0.0, 30.0, -30.0, 19.99, 20.01]
    g1, g2 = orc.gdn_decay(a, A, dt), ref.gdn_decay(a, A, dt)
    assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))
    assert np.array_equal(orc.gdn_beta(b), ref.gdn_beta(b))


@pytest.mark.parametrize("H,D,scale", [(2, 65, 1.0), (16, 128, 128 ** -0.5)])
def test_l2norm_bitwise(orc, ref, rng, H, D, scale):
    x = synth.normal_bf16(rng, (H * D,))
    y1, y2 = orc.gdn_l2norm(x, H, D, scale), ref.gdn_l2norm(x, H, D, scale)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("H,Dk,Dv,T", [(2, 32, 32, 10), (3, 128, 128, 3), (1, 16, 48, 5)])
def test_recurrent_bitwise(orc, ref, rng, H, Dk, Dv, T):
    q = _f32(rng, T * H * Dk, 0.25)
    k = _f32(rng, T * H * Dk, 0.25)
    v = synth.normal_bf16(rng, (T * H * Dv,), 1.5)
    g = (-5.0 * rng.random(T * H)).astype(np.float32)
    beta = bf16_bits(rng.random(T * H).astype(np.float32))
    S0 = _f32(rng, H * Dk * Dv, 0.02)
    S1, S2 = S0.copy(), S0.copy()
    o1 = orc.gdn_recurrent(S1, q, k, v, g, beta, T, H, Dk, Dv)
    o2 = ref.gdn_recurrent(S2, q, k, v, g, beta, T, H, Dk, Dv)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(S1.view(np.uint32), S2.view(np.uint32))
    # step_mt == step at several thread counts (contiguous head partition)
    for nt in (1, 2, 3):
        S3 = S0.copy()
        o3 = np.concatenate([
            orc.gdn_step_mt(S3, q[t * H * Dk:(t + 1) * H * Dk], k[t * H * Dk:(t + 1) * H * Dk],
                            v[t * H * Dv:(t + 1) * H * Dv], g[t * H:(t + 1) * H],
                            beta[t * H:(t + 1) * H], H, Dk, Dv, nthreads=nt)
            for t in range(T)])
        assert np.array_equal(o3.view(np.uint32), o1.view(np.uint32))
        assert np.array_equal(S3.view(np.uint32), S1.view(np.uint32))


@pytest.mark.parametrize("H,D", [(3, 96), (32, 128)])
def test_onorm_bitwise(orc, ref, rng, H, D):
    o = synth.normal_bf16(rng, (H * D,), 1.5)
    z = synth.normal_bf16(rng, (H * D,), 2.0)
    w = synth.normal_bf16(rng, (D,), 0.8)
    assert np.array_equal(orc.gdn_onorm(o, z, w, H, D), ref.gdn_onorm(o, z, w, H, D))


@pytest.mark.parametrize("N", [256, 1023, 2048])
def test_rmsnorm_bitwise(orc, ref, rng, N):
    x = synth.normal_bf16(rng, (N,), 2.0)
    w = synth.normal_bf16(rng, (N,), 0.1)
    assert np.array_equal(orc.attn_rmsnorm(x, w), ref.attn_rmsnorm(x, w))


@pytest.mark.parametrize("pos", [0.0, 1.0, 7.0, 1000.0, 32767.0, 131071.0, 262143.0])
def test_rope_bitwise(orc, ref, rng, pos):
    x = synth.normal_bf16(rng, (256,))
    assert np.array_equal(orc.attn_rope(x, 64, pos), ref.attn_rope(x, 64, pos))


@pytest.mark.parametrize("Tq,Tk,H,Hkv,D", [(6, 6, 4, 2, 64), (7, 7, 3, 1, 65), (2, 37, 16, 2, 256)])
def test_gqa_bitwise(orc, ref, rng, Tq, Tk, H, Hkv, D):
    q = synth.normal_bf16(rng, (Tq * H * D,))
    kc = synth.normal_bf16(rng, (Tk * Hkv * D,))
    vc = synth.normal_bf16(rng, (Tk * Hkv * D,), 1.2)
    scale = np.float32(1.0 / np.sqrt(D))
    o1 = orc.attn_gqa(q, kc, vc, Tq, Tk, H, Hkv, D, scale)
    assert np.array_equal(o1, ref.attn_gqa(q, kc, vc, Tq, Tk, H, Hkv, D, scale))
    assert np.array_equal(o1, orc.attn_gqa_mt(q, kc, vc, Tq, Tk, H, Hkv, D, scale, 3))
    assert np.array_equal(o1, ref.attn_gqa_mt(q, kc, vc, Tq, Tk, H, Hkv, D, scale))


def test_outgate_bitwise(orc, ref, rng):
    o = synth.normal_bf16(rng, (4099,), 1.5)
    gt = synth.normal_bf16(rng, (4099,), 4.0)
    assert np.array_equal(orc.attn_outgate(o, gt), ref.attn_outgate(o, gt))


def test_gdn_mixer_bitwise(orc, ref, rng):
    """Three sequences of 1, 4 and 2 tokens with their own conv/S state at
    the model's dims: oracle mixer == reference ops wired as c/layer.h."""
    dims = synth.GDN_DIMS
    w = synth.gdn_weights(rng)
    cu = np.array([0, 1, 5, 7], np.int32)
    tok = synth.gdn_tokens(rng, 7)
    conv, S = synth.gdn_state(rng, 3)
    c1, S1, c2, S2 = conv.copy(), S.copy(), conv.copy(), S.copy()
    y1 = orc.gdn_mixer(dims, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], c1, S1, nthreads=3)
    y2 = ref.gdn_mixer(dims, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], c2, S2)
    assert np.array_equal(y1, y2)
    assert np.array_equal(c1, c2)
    assert np.array_equal(S1.view(np.uint32), S2.view(np.uint32))


def test_attn_mixer_bitwise(orc, ref, rng):
    """Two sequences (3 new tokens at pos 5, 1 new token at pos 40) over
    their own caches: oracle mixer == reference ops wired as c/layer.h."""
    dims = synth.ATTN_DIMS
    nh, nkv, d = dims[:3]
    w = synth.attn_weights(rng)
    cu = np.array([0, 3, 4], np.int32)
    pos0 = np.array([5, 40], np.int32)
    tok = synth.attn_tokens(rng, 4)
    maxs = 48
    kc = synth.normal_bf16(rng, (2, maxs, nkv, d))
    vc = synth.normal_bf16(rng, (2, maxs, nkv, d))
    k1, v1, k2, v2 = kc.copy(), vc.copy(), kc.copy(), vc.copy()
    stride = maxs * nkv * d
    y1 = orc.attn_mixer(dims, w, cu, pos0, tok["qg"], tok["k"], tok["v"], k1, v1, stride, nthreads=2)
    y2 = ref.attn_mixer(dims, w, cu, pos0, tok["qg"], tok["k"], tok["v"], k2, v2, stride)
    assert np.array_equal(y1, y2)
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


def test_attn_mixer_off_bitwise(orc, ref, rng):
    """The offset-addressed oracle mixer (compact per-sequence caches, as
    the full-size GPU tests use) against the reference ops wired as
    c/layer.h over strided caches; its prep phase gives the captured roped
    q, and outgate(attno, gate) gives y."""
    dims = synth.ATTN_DIMS
    nh, nkv, d = dims[:3]
    w = synth.attn_weights(rng)
    cu = np.array([0, 2, 6, 7], np.int32)
    pos0 = np.array([9, 0, 30], np.int32)
    tok = synth.attn_tokens(rng, 7)
    maxs = 32
    kc = synth.normal_bf16(rng, (3, maxs, nkv, d))
    vc = synth.normal_bf16(rng, (3, maxs, nkv, d))
    k2, v2 = kc.copy(), vc.copy()
    y2 = ref.attn_mixer(dims, w, cu, pos0, tok["qg"], tok["k"], tok["v"], k2, v2, maxs * nkv * d)
    rows = pos0 + np.diff(cu)
    off = np.concatenate([[0], np.cumsum(rows * nkv * d)])
    hk = np.concatenate([kc[s, :rows[s]].reshape(-1) for s in range(3)])
    hv = np.concatenate([vc[s, :rows[s]].reshape(-1) for s in range(3)])
    hk2, hv2 = hk.copy(), hv.copy()
    y1, qf, kf, ao = orc.attn_mixer_off(dims, w, cu, pos0, tok["qg"], tok["k"], tok["v"], hk, hv,
                                        off[:-1], nthreads=3, capture=True)
    assert np.array_equal(y1, y2)
    for s in range(3):
        assert np.array_equal(hk[off[s]:off[s + 1]].reshape(-1, nkv, d), k2[s, :rows[s]])
        assert np.array_equal(hv[off[s]:off[s + 1]].reshape(-1, nkv, d), v2[s, :rows[s]])
    qn = orc.attn_prep_off(dims, w, cu, pos0, tok["qg"], tok["k"], tok["v"], hk2, hv2, off[:-1])
    assert np.array_equal(qn, qf)
    assert np.array_equal(hk2, hk) and np.array_equal(hv2, hv)
    gate = np.ascontiguousarray(tok["qg"].reshape(7, nh, 2 * d)[:, :, d:]).reshape(-1)
    assert np.array_equal(ref.attn_outgate(np.ascontiguousarray(ao.reshape(-1)), gate),
                          y1.reshape(-1))


@pytest.mark.parametrize("M,O,K", [(1, 300, 2048), (4, 129, 4096), (3, 17, 37)])
def test_bf16_gemm_bitwise(orc, ref, rng, M, O, K):
    """The projection restatement against the reference's x86 hot path and
    its scalar anchor (c/bf16.h:178-231, 285-300)."""
    w = synth.normal_bf16(rng, (O, K), 0.05)
    x = synth.normal_bf16(rng, (M, K))
    y = orc.bf16_gemm(w, x)
    assert np.array_equal(y, ref.bf16_gemm(w, x))
    assert np.array_equal(y, ref.bf16_gemm(w, x, hot=False))
    if M == 1:
        assert np.array_equal(y[0], ref.bf16_gemv(w, np.ascontiguousarray(x[0])))
