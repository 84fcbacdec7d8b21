"""Pin the oracle against what the mathematics fixes, independently of the
reference build: float64 truths on odd shapes with the reference's
esc-normalised tolerance |c - gold| <= rel*|gold| + escfrac*esc
(tests/m4a/test_gdn.c:84-95), exact corners (test_gdn.c:278-771,
test_attn.c:190-460), and the RNE narrowing rule checked by a
candidate-distance method over every tie-relevant bit pattern.

Each truth below is written in float64 from the contract formulas
(c/gdn.h:17-75, c/attn.h:16-58), replicating only the bf16 rounding points
the contract names; a dropped term, a swapped operand or a wrong rounding
point fails them.
"""
import numpy as np
import pytest

import synth
from synth import bf16_bits, bf16_f32


def tol_ok(c, gold, esc, rel, escfrac):
    return np.abs(np.asarray(c, np.float64) - gold) <= rel * np.abs(gold) + escfrac * esc + 1e-30


def rnd64(x):
    """Round float64 values through fp32 to bf16 and back (as the truths do)."""
    return bf16_f32(bf16_bits(np.asarray(x, np.float64).astype(np.float32))).astype(np.float64)


def sig64(x):
    return 1.0 / (1.0 + np.exp(-x))


# ---------------------------------------------------------------- RNE rule
def test_bf16_rne_candidate_distance(orc):
    """Every high half with the tie-relevant low halves, plus random bits:
    the result is the nearer of the two bf16 neighbours, ties to even, NaN
    keeps its high half, overflow rounds to inf."""
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    u = (hi[:, None] | lows[None, :]).ravel()
    u = np.concatenate([u, np.random.default_rng(1).integers(0, 2**32, 1 << 22, dtype=np.uint64).astype(np.uint32)])
    x = u.view(np.float32)
    got = orc.bf16_narrow(x)
    nan = np.isnan(x)
    assert np.array_equal(got[nan], (u[nan] >> 16).astype(np.uint16))
    inf = np.isinf(x)
    assert np.array_equal(got[inf], (u[inf] >> 16).astype(np.uint16))
    keep = ~nan & ~inf
    u, x, got = u[keep], x[keep], got[keep]
    lo_code = (u >> 16).astype(np.uint16)             # truncation toward zero
    hi_code = (lo_code.astype(np.uint32) + 1).astype(np.uint16)
    lo = bf16_f32(lo_code).astype(np.float64)
    hi_val = bf16_f32(hi_code).astype(np.float64)
    # the next code above the max finite magnitude is inf; its "distance"
    # is the value 2^128 (RNE overflow rule)
    big = np.isinf(hi_val)
    hi_val = np.where(big, np.sign(lo) * 2.0 ** 128, hi_val)
    xv = x.astype(np.float64)
    dlo, dhi = np.abs(xv - lo), np.abs(hi_val - xv)
    want = np.where(dlo < dhi, lo_code, hi_code)
    tie = dlo == dhi
    want = np.where(tie, np.where(lo_code & 1, hi_code, lo_code), want)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- conv
def conv_truth(x, w, C, T):
    xf = bf16_f32(x).astype(np.float64).reshape(T, C)
    wf = bf16_f32(w).astype(np.float64).reshape(C, 4)
    out = np.zeros((T, C))
    esc = np.zeros((T, C))
    for t in range(T):
        acc = np.zeros(C)
        sc = np.zeros(C)
        for i in range(4):
            ti = t - 3 + i
            if ti < 0:
                continue
            p = wf[:, i] * xf[ti]
            acc += p
            sc += np.abs(p)
        co = rnd64(acc)
        out[t] = co * sig64(co)
        esc[t] = sc
    return out, esc


def test_conv_truth_and_corners(orc, rng):
    C, T = 37, 9
    x = bf16_bits(rng.uniform(-6, 6, T * C).astype(np.float32)).reshape(T, C)
    w = bf16_bits(rng.uniform(-2.8, 2.8, C * 4).astype(np.float32)).reshape(C, 4)
    st = np.zeros(C * 3, np.uint16)
    out = orc.gdn_conv1d(x, w, st)
    tr, esc = conv_truth(x, w, C, T)
    assert tol_ok(bf16_f32(out).reshape(T, C), tr, esc, 0.008, 0.008).all()
    # state == last three pre-conv inputs, exact codes
    assert np.array_equal(st.reshape(C, 3), x[T - 3:].T)
    # zero input -> silu(0) = +0 codes
    z = orc.gdn_conv1d_step(np.zeros(C, np.uint16), w, np.zeros(C * 3, np.uint16))
    assert (z == 0).all()


# ---------------------------------------------------------------- decay / beta
def test_decay_truth_and_corners(orc, rng):
    H = 13
    a = bf16_bits(rng.uniform(-8, 8, H).astype(np.float32))
    A = rng.uniform(-1, 1, H).astype(np.float32)
    dt = rng.uniform(-2, 2, H).astype(np.float32)
    g = orc.gdn_decay(a, A, dt)
    t = bf16_f32(a).astype(np.float64) + dt.astype(np.float64)
    sp = np.where(t > 20, t, np.log1p(np.exp(t)))
    tr = -np.exp(A.astype(np.float64)) * sp
    assert tol_ok(g, tr, 5.0, 2e-6, 2e-7).all()
    # a + dt = 0 -> -exp(A) ln 2 ; a + dt = 25 -> identity branch ; tail
    a2 = bf16_bits(np.array([1.0, 5.0, -25.0], np.float32))
    dt2 = np.array([-1.0, 20.0, 0.0], np.float32)
    A2 = np.array([0.5, 1.25, 0.0], np.float32)
    g2 = orc.gdn_decay(a2, A2, dt2)
    assert abs(g2[0] - (-np.exp(0.5) * np.log(2.0))) <= 1e-6 * np.exp(0.5) * np.log(2.0)
    assert abs(g2[1] - (-np.exp(1.25) * 25.0)) <= 1e-5 * np.exp(1.25) * 25.0
    assert abs(g2[2] - (-np.log1p(np.exp(-25.0)))) <= 1e-6 * np.exp(-25.0)


def test_beta_corners(orc, rng):
    b = bf16_bits(np.array([0.0, 20.0, -20.0], np.float32))
    beta = orc.gdn_beta(b)
    assert beta[0] == 0x3F00 and beta[1] == 0x3F80
    assert bf16_f32(beta[2:3])[0] < 1e-6
    b = bf16_bits(rng.uniform(-10, 10, 257).astype(np.float32))
    tr = sig64(bf16_f32(b).astype(np.float64))
    assert tol_ok(bf16_f32(orc.gdn_beta(b)), tr, 0.02, 0.008, 0.008).all()


# ---------------------------------------------------------------- l2norm
def test_l2norm_truth_and_zero(orc, rng):
    H, D = 2, 65
    x = bf16_bits(rng.uniform(-4, 4, H * D).astype(np.float32))
    y = orc.gdn_l2norm(x, H, D, 1.0)
    xf = bf16_f32(x).astype(np.float64).reshape(H, D)
    tr = xf / np.sqrt((xf * xf).sum(1, keepdims=True) + 1e-6)
    assert tol_ok(y.reshape(H, D), tr, 0.3, 2e-6, 2e-6).all()
    yq = orc.gdn_l2norm(x, H, D, np.float32(D ** -0.5))
    assert tol_ok(yq.reshape(H, D), tr * D ** -0.5, 0.3, 2e-6, 2e-6).all()
    zero = orc.gdn_l2norm(np.zeros(H * 64, np.uint16), H, 64, 1.0)
    assert (zero.view(np.uint32) == 0).all()


# ---------------------------------------------------------------- recurrence
def rec_truth(q, k, v, g, beta, T, H, D):
    """float64 delta rule with propagated error scales (test_gdn.c:488-533
    design): escS tracks |terms| of each state entry, esco of each output."""
    S = np.zeros((H, D, D))
    eS = np.zeros((H, D, D))
    o = np.zeros((T, H, D))
    eo = np.zeros((T, H, D))
    q = q.astype(np.float64).reshape(T, H, D)
    k = k.astype(np.float64).reshape(T, H, D)
    vf = bf16_f32(v).astype(np.float64).reshape(T, H, D)
    bf = bf16_f32(beta).astype(np.float64).reshape(T, H)
    for t in range(T):
        for h in range(H):
            dec = np.exp(float(g[t * H + h]))
            S[h] *= dec
            eS[h] *= dec
            delta = (vf[t, h] - k[t, h] @ S[h]) * bf[t, h]
            upd = np.outer(k[t, h], delta)
            S[h] += upd
            eS[h] += np.abs(upd)
            o[t, h] = q[t, h] @ S[h]
            eo[t, h] = np.abs(q[t, h]) @ np.abs(S[h])
    return S, o, eS, eo


def test_recurrence_truth_and_corners(orc, rng):
    H, D, T = 2, 32, 10
    q = rng.uniform(-1, 1, T * H * D).astype(np.float32)
    k = rng.uniform(-1, 1, T * H * D).astype(np.float32)
    v = bf16_bits(rng.uniform(-6, 6, T * H * D).astype(np.float32))
    g = (-5.0 * rng.random(T * H)).astype(np.float32)
    beta = bf16_bits(rng.random(T * H).astype(np.float32))
    S = np.zeros(H * D * D, np.float32)
    o = orc.gdn_recurrent(S, q, k, v, g, beta, T, H, D, D)
    St, ot, eS, eo = rec_truth(q, k, v, g, beta, T, H, D)
    assert tol_ok(o.reshape(T, H, D), ot, eo, 1e-5, 1e-5).all()
    assert tol_ok(S.reshape(H, D, D), St, eS, 1e-5, 1e-5).all()
    # g = 0, beta = 0 -> S unchanged (bitwise)
    S0 = ((np.arange(D * D) % 7) * 0.25 - 0.75).astype(np.float32)
    S1 = S0.copy()
    q1 = rng.uniform(-1, 1, D).astype(np.float32)
    k1 = rng.uniform(-1, 1, D).astype(np.float32)
    v1 = bf16_bits(rng.uniform(-4, 4, D).astype(np.float32))
    orc.gdn_step(S1, q1, k1, v1, np.zeros(1, np.float32), np.zeros(1, np.uint16), 1, D, D)
    assert np.array_equal(S1.view(np.uint32), S0.view(np.uint32))
    # g = -5 with k = 0 -> exact decay S * expf(-5)
    S2 = S0.copy()
    orc.gdn_step(S2, q1, np.zeros(D, np.float32), np.zeros(D, np.uint16),
                 np.array([-5.0], np.float32), bf16_bits(np.array([0.5], np.float32)), 1, D, D)
    assert np.array_equal(S2, S0 * np.float32(np.exp(-5.0)))   # expf(-5) is the CR value
    # beta = 1 with a unit k: the k-row of S is replaced by v (full replace)
    S3 = S0.copy()
    e0 = np.zeros(D, np.float32)
    e0[3] = 1.0
    orc.gdn_step(S3, q1, e0, v1, np.zeros(1, np.float32), bf16_bits(np.ones(1, np.float32)), 1, D, D)
    assert np.array_equal(S3.reshape(D, D)[3], bf16_f32(v1))


# ---------------------------------------------------------------- onorm
def onorm_truth(o, z, w, H, D):
    of = bf16_f32(o).astype(np.float64).reshape(H, D)
    zf = bf16_f32(z).astype(np.float64).reshape(H, D)
    wf = bf16_f32(w).astype(np.float64)
    rs = 1.0 / np.sqrt((of * of).sum(1, keepdims=True) / D + 1e-6)
    x1 = rnd64(of * rs)
    x2 = rnd64(wf * x1)
    return x2 * (zf * sig64(zf))


def test_onorm_truth_and_corners(orc, rng):
    H, D = 3, 96
    o = bf16_bits(rng.uniform(-6, 6, H * D).astype(np.float32))
    z = bf16_bits(rng.uniform(-8, 8, H * D).astype(np.float32))
    w = bf16_bits(rng.uniform(-3.2, 3.2, D).astype(np.float32))
    y = orc.gdn_onorm(o, z, w, H, D)
    assert tol_ok(bf16_f32(y).reshape(H, D), onorm_truth(o, z, w, H, D), 0.02, 0.008, 0.008).all()
    one = bf16_bits(np.ones(H * D, np.float32))
    y = orc.gdn_onorm(one, bf16_bits(np.full(H * D, 88.0, np.float32)), one[:D].copy(), H, D)
    assert y[0] == bf16_bits(np.array([88.0], np.float32))[0]
    y = orc.gdn_onorm(one, bf16_bits(np.full(H * D, -88.0, np.float32)), one[:D].copy(), H, D)
    assert (np.abs(bf16_f32(y)) <= 1e-30).all()


# ---------------------------------------------------------------- attention
def test_rmsnorm_truth_and_zero(orc, rng):
    N = 2048
    x = bf16_bits(rng.uniform(-8, 8, N).astype(np.float32))
    w = bf16_bits(rng.uniform(-0.4, 0.4, N).astype(np.float32))
    y = orc.attn_rmsnorm(x, w)
    xf = bf16_f32(x).astype(np.float64)
    tr = rnd64(xf / np.sqrt((xf * xf).sum() / N + 1e-6) * (1.0 + bf16_f32(w)))
    assert tol_ok(bf16_f32(y), tr, 0.02, 0.008, 0.008).all()
    assert (orc.attn_rmsnorm(np.zeros(N, np.uint16), w) == 0).all()


@pytest.mark.parametrize("pos", [0.0, 1.0, 7.0, 1000.0, 131071.0, 262143.0])
def test_rope_truth(orc, rng, pos):
    D, rot = 256, 64
    R = rot // 2
    x = bf16_bits(rng.uniform(-4, 4, D).astype(np.float32))
    y = orc.attn_rope(x, rot, pos)
    if pos == 0.0:
        assert np.array_equal(y, x)        # cos 0 = 1, sin 0 = 0 exactly
    assert np.array_equal(y[rot:], x[rot:])  # pass-through dims copied
    # cos/sin codes: host table vs float64 angles (the reference allows a
    # libm flip class; at these positions at most 1% of codes may differ)
    i = np.arange(R)
    invf = (1.0 / np.power(1e7, 2.0 * i / rot)).astype(np.float32)
    ang = (np.float32(pos) * invf).astype(np.float64)
    cs = orc.rope_table(pos, rot)
    flips = np.sum(cs[:R] != bf16_bits(np.cos(ang).astype(np.float32))) + \
        np.sum(cs[R:] != bf16_bits(np.sin(ang).astype(np.float32)))
    assert flips <= max(1, rot // 100)
    c = bf16_f32(cs[:R]).astype(np.float64)
    s = bf16_f32(cs[R:]).astype(np.float64)
    xf = bf16_f32(x).astype(np.float64)
    lo, hi = xf[:R], xf[R:rot]
    t0 = rnd64(rnd64(lo * c) + rnd64(-hi * s))
    t1 = rnd64(rnd64(hi * c) + rnd64(lo * s))
    got = bf16_f32(y).astype(np.float64)
    assert tol_ok(got[:R], t0, 0.02, 0.008, 0.008).all()
    assert tol_ok(got[R:rot], t1, 0.02, 0.008, 0.008).all()


def gqa_row_truth(qh, kc, vc, Hkv, D, scale, p, hk):
    """float64 restatement with the bf16 rounding points replicated
    (tests/m4a/test_attn.c:270-306 design)."""
    qf = bf16_f32(qh).astype(np.float64)
    K = bf16_f32(kc).astype(np.float64).reshape(-1, Hkv, D)[: p + 1, hk]
    V = bf16_f32(vc).astype(np.float64).reshape(-1, Hkv, D)[: p + 1, hk]
    A = rnd64(rnd64(K @ qf) * scale)
    e = np.exp(A - A.max())
    P = rnd64(e / e.sum())
    return P @ V, np.abs(P) @ np.abs(V)


def test_gqa_truth_and_decode(orc, rng):
    D, T, H, Hkv = 65, 7, 3, 1
    q = bf16_bits(rng.uniform(-4, 4, T * H * D).astype(np.float32))
    kc = bf16_bits(rng.uniform(-4, 4, T * Hkv * D).astype(np.float32))
    vc = bf16_bits(rng.uniform(-4.8, 4.8, T * Hkv * D).astype(np.float32))
    scale = np.float32(1.0 / np.sqrt(D))
    o = orc.attn_gqa(q, kc, vc, T, T, H, Hkv, D, scale)
    for t in range(T):
        for h in range(H):
            tr, esc = gqa_row_truth(q[(t * H + h) * D:(t * H + h + 1) * D], kc, vc, Hkv, D,
                                    float(scale), t, h // (H // Hkv))
            got = bf16_f32(o[(t * H + h) * D:(t * H + h + 1) * D])
            assert tol_ok(got, tr, esc, 0.008, 0.008).all()
    # decode == last row of the full recompute, bitwise
    od = orc.attn_gqa(q[(T - 1) * H * D:].copy(), kc, vc, 1, T, H, Hkv, D, scale)
    assert np.array_equal(od, o[(T - 1) * H * D:])


def test_outgate_corners(orc, rng):
    o = bf16_bits(rng.uniform(-6, 6, 3).astype(np.float32))
    gate = bf16_bits(np.array([0.0, 20.0, -20.0], np.float32))
    y = orc.attn_outgate(o, gate)
    assert y[0] == bf16_bits(np.array([bf16_f32(o[:1])[0] * np.float32(0.5)], np.float32))[0]
    assert y[1] == o[1]
    assert abs(bf16_f32(y[2:3])[0]) < 1e-6 * (abs(bf16_f32(o[2:3])[0]) + 1e-6)


def test_gemm_truth_and_corners(orc, rng):
    """Projections (c/bf16.h:285-300): against the float64 sum within the
    fp32 accumulation bound (K 2^-24 sum|w x|) plus the final rounding; a
    permutation matrix returns x's codes exactly (catches a transposed or
    shifted index); K = 0 gives +0; sign symmetry is exact."""
    M, O, K = 3, 64, 1024
    w = synth.normal_bf16(rng, (O, K), 0.05)
    x = synth.normal_bf16(rng, (M, K))
    y = orc.bf16_gemm(w, x)
    wf, xf = bf16_f32(w).astype(np.float64), bf16_f32(x).astype(np.float64)
    gold = xf @ wf.T
    esc = np.abs(xf) @ np.abs(wf).T
    assert tol_ok(bf16_f32(y), gold, esc, 2.0 ** -8, K * 2.0 ** -24).all()
    perm = rng.permutation(K)[:O]
    P = np.zeros((O, K), np.uint16)
    P[np.arange(O), perm] = 0x3F80                      # 1.0
    assert np.array_equal(orc.bf16_gemm(P, x), x[:, perm])
    assert np.array_equal(orc.bf16_gemm(w ^ np.uint16(0x8000), x), y ^ np.uint16(0x8000))
    z = orc.bf16_gemm(np.zeros((5, 0), np.uint16), np.zeros((2, 0), np.uint16))
    assert z.shape == (2, 5) and np.all(z == 0)
