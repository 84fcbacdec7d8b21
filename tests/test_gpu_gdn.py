"""GPU parity: Gated DeltaNet ops through the C ABI against the oracle.

Drop-in ops keep the reference's summation order, so outputs must be
bit-identical to the oracle except where a libm ulp (expf/log1pf in the
gates, which the GPU evaluates correctly rounded) crosses a rounding
boundary: bf16 outputs within 1 ulp and 2e-3 relative (tests/numerics.py),
fp32 outputs within 1e-4 relative, with the exact-match fraction reported.
The fused decode is held to the same bar at BASELINE config 0 (B=1), at
B=64, and on ragged multi-token verify batches (config 4's shape).
"""
import numpy as np
import pytest

import synth
from numerics import assert_bf16_close, assert_state_close, f32_stats

pytestmark = pytest.mark.gpu


def _f32(rng, n, s=1.0):
    return rng.standard_normal(n, dtype=np.float32) * np.float32(s)


@pytest.mark.parametrize("C,T", [(37, 9), (8192, 1), (8192, 64)])
def test_conv1d(hip, orc, rng, C, T):
    x = synth.normal_bf16(rng, (T, C), 1.5)
    w = synth.normal_bf16(rng, (C, 4), 0.7)
    st = synth.normal_bf16(rng, (C * 3,))
    s1, s2 = st.copy(), st.copy()
    assert_bf16_close(hip.gdn_conv1d(x, w, s1), orc.gdn_conv1d(x, w, s2), what="conv")
    assert np.array_equal(s1, s2)          # state = exact input codes


def _silu_bf16_reference(codes):
    """rnd(co * sigmoid(co)) with the reference's sigmoid (exp correctly
    rounded to fp32, fp32 add, divide and product; c/gdn.h:19-33)."""
    co = (codes.astype(np.uint32) << 16).view(np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-co.astype(np.float64)).astype(np.float32)
        sg = np.float32(1.0) / (np.float32(1.0) + e)
    p = (co * sg).view(np.uint32)
    return ((p + 0x7FFF + ((p >> 16) & 1)) >> 16).astype(np.uint16)


def test_conv1d_silu_every_code(hip):
    """The conv's SiLU over every finite bf16 code (taps 0,0,0,1 on a zero
    state pass the input code through the sum unchanged), bit-exact: its
    fp32 fast path must hand every near-midpoint product to the reference
    formula."""
    codes = np.arange(65536, dtype=np.uint32)
    finite = ((codes >> 7) & 0xFF) != 0xFF
    x = codes[finite].astype(np.uint16)
    x = x[x != 0x8000][None, :]             # -0 sums to +0
    C = x.shape[1]
    w = np.tile(np.array([0, 0, 0, 0x3F80], np.uint16), (C, 1))
    st = np.zeros(C * 3, np.uint16)
    out = hip.gdn_conv1d(x, w, st)
    exp = _silu_bf16_reference(x[0])
    bad = np.flatnonzero(out[0] != exp)
    assert bad.size == 0, f"{bad.size} codes differ, e.g. {[(hex(x[0][i]), hex(out[0][i]), hex(exp[i])) for i in bad[:5]]}"


def test_decay_beta(hip, orc, rng):
    H = 4099
    a = synth.normal_bf16(rng, (H,), 3.0)
    b = synth.normal_bf16(rng, (H,), 6.0)
    A = rng.uniform(-1, 2.7, H).astype(np.float32)
    dt = _f32(rng, H, 4.0)
    g1, g2 = hip.gdn_decay(a, A, dt), orc.gdn_decay(a, A, dt)
    st = f32_stats(g1, g2)
    assert st["rel"] <= 1e-6, st
    assert_bf16_close(hip.gdn_beta(b), orc.gdn_beta(b), what="beta")
    corner = synth.bf16_bits(np.array([0.0, 20.0], np.float32))
    assert list(hip.gdn_beta(corner)) == [0x3F00, 0x3F80]


@pytest.mark.parametrize("H,D,scale", [(2, 65, 1.0), (16, 128, 128 ** -0.5)])
def test_l2norm_bitwise(hip, orc, rng, H, D, scale):
    x = synth.normal_bf16(rng, (H * D,))
    y1, y2 = hip.gdn_l2norm(x, H, D, scale), orc.gdn_l2norm(x, H, D, scale)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("H,Dk,Dv,T", [(2, 32, 32, 10), (32, 128, 128, 4), (1, 16, 48, 5)])
def test_recurrent(hip, orc, rng, H, Dk, Dv, T):
    q = _f32(rng, T * H * Dk, 0.25)
    k = _f32(rng, T * H * Dk, 0.25)
    v = synth.normal_bf16(rng, (T * H * Dv,), 1.5)
    g = (-5.0 * rng.random(T * H)).astype(np.float32)
    beta = synth.bf16_bits(rng.random(T * H).astype(np.float32))
    S0 = _f32(rng, H * Dk * Dv, 0.02)
    S1, S2 = S0.copy(), S0.copy()
    o1 = hip.gdn_recurrent(S1, q, k, v, g, beta, T, H, Dk, Dv)
    o2 = orc.gdn_recurrent(S2, q, k, v, g, beta, T, H, Dk, Dv)
    assert f32_stats(o1, o2)["rel"] <= 1e-4
    assert_state_close(S1, S2, what="recurrent S")
    # step == recurrent token by token, on the GPU too
    S3 = S0.copy()
    o3 = np.concatenate([hip.gdn_step(S3, q[t * H * Dk:(t + 1) * H * Dk], k[t * H * Dk:(t + 1) * H * Dk],
                                      v[t * H * Dv:(t + 1) * H * Dv], g[t * H:(t + 1) * H],
                                      beta[t * H:(t + 1) * H], H, Dk, Dv) for t in range(T)])
    assert np.array_equal(o3.view(np.uint32), o1.view(np.uint32))
    assert np.array_equal(S3.view(np.uint32), S1.view(np.uint32))


def test_recurrent_corners(hip, rng):
    D = 32
    S0 = ((np.arange(D * D) % 7) * 0.25 - 0.75).astype(np.float32)
    S1 = S0.copy()
    q1 = _f32(rng, D)
    k1 = _f32(rng, D)
    v1 = synth.normal_bf16(rng, (D,))
    hip.gdn_step(S1, q1, k1, v1, np.zeros(1, np.float32), np.zeros(1, np.uint16), 1, D, D)
    assert np.array_equal(S1.view(np.uint32), S0.view(np.uint32))
    S2 = S0.copy()
    hip.gdn_step(S2, q1, np.zeros(D, np.float32), np.zeros(D, np.uint16),
                 np.array([-5.0], np.float32), synth.bf16_bits(np.array([0.5], np.float32)), 1, D, D)
    assert np.array_equal(S2, S0 * np.float32(np.exp(-5.0)))


@pytest.mark.parametrize("H,D", [(3, 96), (32, 128)])
def test_onorm(hip, orc, rng, H, D):
    o = synth.normal_bf16(rng, (H * D,), 1.5)
    z = synth.normal_bf16(rng, (H * D,), 2.0)
    w = synth.normal_bf16(rng, (D,), 0.8)
    assert_bf16_close(hip.gdn_onorm(o, z, w, H, D), orc.gdn_onorm(o, z, w, H, D), what="onorm")


# ---------------------------------------------------------------- fused decode
def _run_decode(hip, orc, rng, cu, zero_state=False):
    import torch
    dims = synth.GDN_DIMS
    B = len(cu) - 1
    T = int(cu[-1])
    w = synth.gdn_weights(rng)
    tok = synth.gdn_tokens(rng, T)
    conv, S = synth.gdn_state(rng, B, zero=zero_state)
    # oracle
    c_o, S_o = conv.copy(), S.copy()
    y_o, tr = orc.gdn_mixer(dims, w, np.asarray(cu, np.int32), tok["qkv"], tok["z"], tok["a"],
                            tok["b"], c_o, S_o, trace=True)
    # GPU (tier 2, device resident)
    dev = torch.device("cuda")
    tw = {k: torch.from_numpy(v.view(np.int16) if v.dtype == np.uint16 else v).to(dev)
          for k, v in w.items()}
    layer = hip.gdn_layer(dims, tw)
    t = {k: torch.from_numpy(v.view(np.int16)).to(dev) for k, v in tok.items()}
    dconv = torch.from_numpy(conv.view(np.int16)).to(dev)
    dS_ref = torch.from_numpy(S).to(dev)
    dS = torch.empty_like(dS_ref)
    hip.gdn_state_pack(dS_ref, dS)            # reference layout -> device layout
    y = torch.empty((T, dims[1] * dims[3]), dtype=torch.int16, device=dev)
    hip.gdn_decode(layer, cu, t["qkv"], t["z"], t["a"], t["b"], dconv, dS, y)
    hip.gdn_state_unpack(dS, dS_ref)
    torch.cuda.synchronize()
    y_h = y.cpu().numpy().view(np.uint16)
    st = assert_bf16_close(y_h, y_o, what="gdn_decode y")
    assert np.array_equal(dconv.cpu().numpy().view(np.uint16), c_o)
    e = assert_state_close(dS_ref.cpu().numpy(), S_o, what="gdn_decode S")
    return st, e


def test_gdn_decode_config0(hip, orc):
    """one layer, one decode step, batch 1, prior state."""
    st, e = _run_decode(hip, orc, np.random.default_rng(20260829), [0, 1])
    print(f"config0 y: {st} state rel {e:.3g}")


@pytest.mark.parametrize("k", [[1, 1, 1], [1, 0, 1, 1, 1, 1, 1, 1, 1], [1] * 8])
def test_gdn_decode_small_batches(hip, orc, k):
    """One token per sequence at small batch sizes (the latency-oriented
    one-token kernel: up to 8 sequences of 16 K heads), an empty sequence
    included."""
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    st, e = _run_decode(hip, orc, np.random.default_rng(len(k)), cu)
    print(f"B={len(k)} y: {st} state rel {e:.3g}")


def test_gdn_decode_batch64(hip, orc):
    """Config 0 at batch 64 (the HBM-bound decode shape)."""
    cu = np.arange(65, dtype=np.int32)
    st, e = _run_decode(hip, orc, np.random.default_rng(64), cu)
    print(f"B=64 y: {st} state rel {e:.3g}")


def test_gdn_decode_ragged_verify(hip, orc):
    """Config 4's GDN shape: each sequence verifies 1..4 tokens."""
    rng = np.random.default_rng(4)
    k = rng.integers(1, 5, 9)
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    _run_decode(hip, orc, rng, cu)


@pytest.mark.parametrize("kmax", [1, 4, 9])
def test_gdn_decode_many_items(hip, orc, kmax):
    """More (sequence, K head) items than compute units, so each persistent
    workgroup carries its pipeline across many items: 200 sequences of
    0..kmax tokens (empty ones included). kmax 1, 4 and 9 take the
    one-token, the up-to-four-token and the general token loop."""
    rng = np.random.default_rng(100 + kmax)
    k = rng.integers(0, kmax + 1, 200)
    k[rng.integers(0, 200)] = kmax
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    _run_decode(hip, orc, rng, cu)


def test_gdn_decode_zero_state_long(hip, orc):
    """A 32-token single sequence from zero state: decode stepping through
    a prefill-length span keeps matching the sequential recurrence."""
    _run_decode(hip, orc, np.random.default_rng(7), [0, 32], zero_state=True)


def test_state_pack_roundtrip(hip):
    """pack then unpack is the identity, and pack places S[i][j] where the
    documented formula says (include/apus_hip.h)."""
    import torch
    n = 3
    S = torch.arange(n * 128 * 128, dtype=torch.float32, device="cuda").reshape(n, 128, 128)
    P = torch.empty_like(S)
    U = torch.empty_like(S)
    hip.gdn_state_pack(S, P)
    hip.gdn_state_unpack(P, U)
    torch.cuda.synchronize()
    assert torch.equal(U, S)
    Ph = P.cpu().numpy().reshape(n, -1)
    for (m, i, j) in [(0, 0, 0), (1, 5, 70), (2, 127, 127), (0, 64, 63)]:
        off = ((j // 64 * 32 + i // 4) * 64 + j % 64) * 4 + i % 4
        assert Ph[m, off] == float(m * 16384 + i * 128 + j)


def test_gdn_decode_into_rollback(hip, orc):
    """Out-of-place verify plus rollback (the device form of the reference's
    MTP snapshot/restore, c/mtp.h:36-75): every sequence verifies 4 tokens
    from the snapshot set into the output set, then the sequences that
    rejected a draft re-feed their accepted prefix from the same snapshot.
    The output set must equal an in-place decode of the accepted prefixes
    (same kernel, so bitwise), the snapshot must be unchanged, fully
    accepted sequences keep their verify state, and the verify outputs
    match the oracle."""
    import torch
    rng = np.random.default_rng(36)
    dims = synth.GDN_DIMS
    B, k = 12, 4
    w = synth.gdn_weights(rng)
    cu = np.arange(0, (B + 1) * k, k, dtype=np.int32)
    tok = synth.gdn_tokens(rng, B * k)
    conv, S = synth.gdn_state(rng, B)
    acc = rng.integers(1, k + 1, B)            # accepted tokens per sequence
    acc[0], acc[1] = k, 1
    dev = torch.device("cuda")
    tw = {n: torch.from_numpy(v.view(np.int16) if v.dtype == np.uint16 else v).to(dev)
          for n, v in w.items()}
    layer = hip.gdn_layer(dims, tw)
    t = {n: torch.from_numpy(v.view(np.int16)).to(dev) for n, v in tok.items()}
    vd = dims[1] * dims[3]
    c_in = torch.from_numpy(conv.view(np.int16)).to(dev)
    S_ref = torch.from_numpy(S).to(dev)
    S_in = torch.empty_like(S_ref)
    hip.gdn_state_pack(S_ref, S_in)
    c_snap, S_snap = c_in.clone(), S_in.clone()
    c_out, S_out = torch.zeros_like(c_in), torch.zeros_like(S_in)
    y = torch.empty((B * k, vd), dtype=torch.int16, device=dev)
    # verify: all k tokens, snapshot -> output set
    hip.gdn_decode_into(layer, cu, t["qkv"], t["z"], t["a"], t["b"], c_in, S_in, c_out, S_out, y)
    c_o, S_o = conv.copy(), S.copy()
    y_o = orc.gdn_mixer(dims, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], c_o, S_o)
    torch.cuda.synchronize()
    assert_bf16_close(y.cpu().numpy().view(np.uint16), y_o, what="verify y")
    assert torch.equal(c_in, c_snap) and torch.equal(S_in, S_snap), "snapshot modified"
    S_full = S_out.clone()
    # rollback: re-feed the accepted prefix of rejected sequences only
    rej = [s for s in range(B) if acc[s] < k]
    ncu = np.zeros(B + 1, np.int32)
    rows = []
    for s in range(B):
        n = acc[s] if acc[s] < k else 0
        ncu[s + 1] = ncu[s] + n
        rows += list(range(s * k, s * k + n))
    idx = torch.tensor(rows, device=dev, dtype=torch.long)
    y2 = torch.empty((len(rows), vd), dtype=torch.int16, device=dev)
    hip.gdn_decode_into(layer, ncu, t["qkv"][idx].contiguous(), t["z"][idx].contiguous(),
                        t["a"][idx].contiguous(), t["b"][idx].contiguous(),
                        c_in, S_in, c_out, S_out, y2)
    # expected: in-place decode of every accepted prefix from the snapshot
    pcu = np.concatenate([[0], np.cumsum(acc)]).astype(np.int32)
    prow = torch.tensor([s * k + i for s in range(B) for i in range(acc[s])],
                        device=dev, dtype=torch.long)
    c_e, S_e = c_snap.clone(), S_snap.clone()
    y3 = torch.empty((int(pcu[-1]), vd), dtype=torch.int16, device=dev)
    hip.gdn_decode(layer, pcu, t["qkv"][prow].contiguous(), t["z"][prow].contiguous(),
                   t["a"][prow].contiguous(), t["b"][prow].contiguous(), c_e, S_e, y3)
    torch.cuda.synchronize()
    assert torch.equal(c_out, c_e), "rolled-back conv state"
    assert torch.equal(S_out, S_e), "rolled-back S"
    assert torch.equal(c_in, c_snap) and torch.equal(S_in, S_snap), "snapshot modified"
    for s in range(B):
        if acc[s] == k:
            assert torch.equal(S_out[s], S_full[s])
    # the re-fed rows' outputs equal the prefix decode's
    prow_l = prow.tolist()
    pos = {r: i for i, r in enumerate(prow_l)}
    sel = torch.tensor([pos[r] for r in rows], device=dev, dtype=torch.long)
    assert torch.equal(y2, y3[sel])
    assert rej, "seed gives at least one rejected sequence"


def test_gdn_decode_into_rejects_partial_overlap(hip):
    """In/out state sets must be the same buffer or disjoint."""
    import torch
    rng = np.random.default_rng(1)
    dims = synth.GDN_DIMS
    dev = torch.device("cuda")
    w = synth.gdn_weights(rng)
    tw = {n: torch.from_numpy(v.view(np.int16) if v.dtype == np.uint16 else v).to(dev)
          for n, v in w.items()}
    layer = hip.gdn_layer(dims, tw)
    tok = synth.gdn_tokens(rng, 2)
    t = {n: torch.from_numpy(v.view(np.int16)).to(dev) for n, v in tok.items()}
    conv, S = synth.gdn_state(rng, 2)
    c = torch.from_numpy(conv.view(np.int16)).to(dev)
    Sb = torch.zeros((3 * dims[1], 128, 128), dtype=torch.float32, device=dev)
    y = torch.empty((2, dims[1] * dims[3]), dtype=torch.int16, device=dev)
    with pytest.raises(RuntimeError, match="disjoint"):
        hip.gdn_decode_into(layer, [0, 1, 2], t["qkv"], t["z"], t["a"], t["b"],
                            c, Sb[:2 * dims[1]], c.clone(), Sb[dims[1]:], y)


def test_gdn_decode_tokens_equal_steps(hip):
    """The reference's step-loop invariance (recurrent == step loop,
    bitwise; tests/m4a): sequences decoding 9, 4 and 1 tokens in one call
    leave the same outputs, conv state and recurrent state, bit for bit, as
    the same tokens fed one decode call per token."""
    import torch
    rng = np.random.default_rng(91)
    dims = synth.GDN_DIMS
    k = [9, 4, 1]
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    B, T = len(k), int(cu[-1])
    w = synth.gdn_weights(rng)
    tok = synth.gdn_tokens(rng, T)
    conv, S = synth.gdn_state(rng, B)
    dev = torch.device("cuda")
    tw = {n: torch.from_numpy(v.view(np.int16) if v.dtype == np.uint16 else v).to(dev)
          for n, v in w.items()}
    layer = hip.gdn_layer(dims, tw)
    t = {n: torch.from_numpy(v.view(np.int16)).to(dev) for n, v in tok.items()}
    dS0 = torch.empty((B,) + S.shape[1:], dtype=torch.float32, device=dev)
    hip.gdn_state_pack(torch.from_numpy(S).to(dev), dS0)
    vd = dims[1] * dims[3]
    # one call
    c1, S1 = torch.from_numpy(conv.view(np.int16)).to(dev), dS0.clone()
    y1 = torch.empty((T, vd), dtype=torch.int16, device=dev)
    hip.gdn_decode(layer, cu, t["qkv"], t["z"], t["a"], t["b"], c1, S1, y1)
    # one call per token of each sequence
    c2, S2 = torch.from_numpy(conv.view(np.int16)).to(dev), dS0.clone()
    y2 = torch.empty((T, vd), dtype=torch.int16, device=dev)
    for s in range(B):
        for j in range(int(cu[s]), int(cu[s + 1])):
            hip.gdn_decode(layer, [0, 1], t["qkv"][j:j + 1], t["z"][j:j + 1], t["a"][j:j + 1],
                           t["b"][j:j + 1], c2[s:s + 1], S2[s:s + 1], y2[j:j + 1])
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "outputs"
    assert torch.equal(c1, c2), "conv state"
    assert torch.equal(S1, S2), "recurrent state"
