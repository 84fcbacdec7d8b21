"""GPU parity at BASELINE.json's full configuration sizes, against the oracle.

- config 2: gated-GQA decode, all 64 sequences with a 32768-token cache;
- config 3: gated-GQA causal prefill at T=8192 from position 0; the whole
  cache fill is checked bit-exact; the outputs of every head on 17 sampled
  blocks of 64 query rows are recomputed by the oracle's ordered GQA rows
  over the full causal key range, and all 8192 rows of every head against
  a float64 torch reference with the reference's rounding points;
- config 4: the hybrid 3 GDN + 1 GQA decode block on the benchmark's own
  ragged batch (128 sequences, log-normal contexts mu = ln 4096, sigma = 1,
  up to 36066 cached tokens, 1..4 verify tokens each), every layer against
  the oracle;
- batches above the 224 sequences whose metadata travels by value in the
  attention kernels (B = 260) for decode and prefill, and a GDN decode batch
  above its 480-sequence inline limit.

Bars (tests/numerics.py): GQA outputs |c - r| <= 2e-3 (|r| + esc) per
element (esc = sum_j P_j |V_jd|, the reference's esc form) or 2 bf16 ulps,
and 2e-3 normwise; appended cache rows bit-exact; GDN outputs within 1 bf16
ulp and 2e-3 normwise, conv state bit-exact, recurrent state within 1e-4.
Cache contents are drawn on the device (torch, bf16 by round-to-nearest-
even) and copied to the host for the oracle, so gigabyte-sized caches cost
seconds.
"""
import numpy as np
import pytest

import synth
from attn_util import attn_esc_rows
from numerics import assert_bf16_close, assert_bf16_esc, assert_state_close

pytestmark = pytest.mark.gpu

NH, NKV, D, ROT, THETA = synth.ATTN_DIMS
NTHREADS = 16


def _td(torch, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to("cuda")


def _h(t):
    return t.cpu().numpy().view(np.uint16)


def _randn_codes(torch, g, shape):
    return (torch.randn(shape, generator=g, device="cuda")).to(torch.bfloat16).view(torch.int16)


def _device_caches(torch, g, B, rows, max_seq):
    """Per sequence s, rows[s] random cache rows (reference layout
    [rows, nkv, d]) packed into the device flat layout; returns the device
    caches and the host copies concatenated with their element offsets."""
    dk = torch.zeros((B, NKV, max_seq, D), dtype=torch.int16, device="cuda")
    dv = torch.zeros((B, NKV, max_seq // 32, D, 32), dtype=torch.int16, device="cuda")
    off = np.zeros(B + 1, np.int64)
    off[1:] = np.cumsum(np.asarray(rows, np.int64) * NKV * D)
    hk = np.empty(int(off[-1]), np.uint16)
    hv = np.empty(int(off[-1]), np.uint16)
    return dk, dv, off, hk, hv


def _fill_caches(hip, torch, g, B, ctx, rows, max_seq):
    dk, dv, off, hk, hv = _device_caches(torch, g, B, rows, max_seq)
    for s in range(B):
        kr = _randn_codes(torch, g, (int(rows[s]), NKV, D))
        vr = _randn_codes(torch, g, (int(rows[s]), NKV, D))
        if ctx[s]:
            hip.attn_cache_pack(kr, vr, int(ctx[s]), NKV, D, dk[s], dv[s], max_seq)
        hk[off[s]:off[s + 1]] = _h(kr).reshape(-1)
        hv[off[s]:off[s + 1]] = _h(vr).reshape(-1)
    torch.cuda.synchronize()
    return dk, dv, off, hk, hv


def _check_appended(dk, dv, hk, hv, off, pos0, k, max_seq=None, hip=None):
    """The rows the mixer appended (positions pos0[s] .. pos0[s]+k[s]-1)
    equal the oracle's, bit for bit (read back through the cache unpack)."""
    import torch
    for s in range(len(pos0)):
        p0, p1 = int(pos0[s]), int(pos0[s]) + int(k[s])
        rk = torch.empty((p1, NKV, D), dtype=torch.int16, device="cuda")
        rv = torch.empty_like(rk)
        hip.attn_cache_unpack(dk[s], dv[s], p1, NKV, D, max_seq, rk, rv)
        torch.cuda.synchronize()
        Ko = hk[off[s]:off[s + 1]].reshape(-1, NKV, D)[p0:p1]
        Vo = hv[off[s]:off[s + 1]].reshape(-1, NKV, D)[p0:p1]
        assert np.array_equal(_h(rk[p0:p1]), Ko), f"k cache rows of sequence {s}"
        assert np.array_equal(_h(rv[p0:p1]), Vo), f"v cache rows of sequence {s}"


def _attn_decode_case(hip, orc, seed, ctx, k, tag):
    """B sequences with ctx[s] cached tokens verifying k[s] new ones,
    through apus_hip_attn_decode, against the oracle mixer."""
    import torch
    B = len(ctx)
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    pos0 = np.asarray(ctx, np.int32)
    T = int(cu[-1])
    rows = pos0 + np.asarray(k, np.int32)
    max_seq = int(-(-int(rows.max()) // 32) * 32)
    print(f"[{tag}] B={B} T={T} ctx mean {pos0.mean():.0f} max {pos0.max()} "
          f"max_seq={max_seq}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(seed)
    rng = np.random.default_rng(seed)
    dk, dv, off, hk, hv = _fill_caches(hip, torch, g, B, pos0, rows, max_seq)
    w = synth.attn_weights(rng)
    tok = synth.attn_tokens(rng, T)
    layer = hip.attn_layer(synth.ATTN_DIMS, {n: _td(torch, a) for n, a in w.items()})
    t = {n: _td(torch, a) for n, a in tok.items()}
    y = torch.empty((T, NH * D), dtype=torch.int16, device="cuda")
    hip.attn_decode(layer, cu, pos0, t["qg"], t["k"], t["v"], dk, dv, max_seq, y)
    torch.cuda.synchronize()
    y_o, qf, _, _ = orc.attn_mixer_off(synth.ATTN_DIMS, w, cu, pos0, tok["qg"], tok["k"],
                                       tok["v"], hk, hv, off[:-1], nthreads=NTHREADS,
                                       capture=True)
    _check_appended(dk, dv, hk, hv, off, pos0, k, max_seq, hip)
    esc = np.concatenate([
        attn_esc_rows(qf[cu[s]:cu[s + 1]], hk[off[s]:off[s + 1]].reshape(-1, NKV, D),
                      hv[off[s]:off[s + 1]].reshape(-1, NKV, D),
                      pos0[s] + np.arange(k[s]), NH, NKV, D) for s in range(B)])
    st = assert_bf16_esc(_h(y), y_o, esc, ulps=2, what=f"{tag} y")
    print(f"[{tag}] {st}", flush=True)


def test_config2_full(hip, orc):
    """64 sequences x 32768 keys (32767 cached + the new
    token), one new token each."""
    _attn_decode_case(hip, orc, 21, np.full(64, 32767, np.int32), np.ones(64, np.int32),
                      "config2 64x32K")


def test_attn_decode_b260(hip, orc):
    """260 sequences (device-side metadata) with ragged contexts and 1..4
    verify tokens."""
    rng = np.random.default_rng(22)
    ctx = rng.integers(1, 700, 260).astype(np.int32)
    k = rng.integers(1, 5, 260).astype(np.int32)
    _attn_decode_case(hip, orc, 22, ctx, k, "attn decode B=260")


def test_attn_prefill_b260(hip, orc):
    """260 ragged prefill sequences (1..40 new tokens after 0..100 cached):
    the device-metadata path of the prefill."""
    import torch
    rng = np.random.default_rng(23)
    B = 260
    ctx = rng.integers(0, 100, B).astype(np.int32)
    k = rng.integers(1, 41, B).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    T = int(cu[-1])
    rows = ctx + k
    max_seq = int(-(-int(rows.max()) // 32) * 32)
    print(f"[attn prefill B=260] T={T} max_seq={max_seq}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(23)
    dk, dv, off, hk, hv = _fill_caches(hip, torch, g, B, ctx, rows, max_seq)
    w = synth.attn_weights(rng)
    tok = synth.attn_tokens(rng, T)
    layer = hip.attn_layer(synth.ATTN_DIMS, {n: _td(torch, a) for n, a in w.items()})
    t = {n: _td(torch, a) for n, a in tok.items()}
    y = torch.empty((T, NH * D), dtype=torch.int16, device="cuda")
    hip.attn_prefill(layer, cu, ctx, t["qg"], t["k"], t["v"], dk, dv, max_seq, y)
    torch.cuda.synchronize()
    y_o, qf, _, _ = orc.attn_mixer_off(synth.ATTN_DIMS, w, cu, ctx, tok["qg"], tok["k"],
                                       tok["v"], hk, hv, off[:-1], nthreads=NTHREADS,
                                       capture=True)
    _check_appended(dk, dv, hk, hv, off, ctx, k, max_seq, hip)
    esc = np.concatenate([
        attn_esc_rows(qf[cu[s]:cu[s + 1]], hk[off[s]:off[s + 1]].reshape(-1, NKV, D),
                      hv[off[s]:off[s + 1]].reshape(-1, NKV, D),
                      ctx[s] + np.arange(k[s]), NH, NKV, D) for s in range(B)])
    st = assert_bf16_esc(_h(y), y_o, esc, ulps=2, what="attn prefill B=260 y")
    print(f"[attn prefill B=260] {st}", flush=True)


# 17 blocks of 64 query rows over the whole prompt (every 8th 64-row tile
# and its odd 32-row offsets, so both halves of the kernel's 32-token query
# tiles are sampled): the first tile, rows just past every 2048 boundary,
# a block straddling one (2016..2079), and the last diagonal tile, with
# all 16 heads (both kv heads) of each row checked.
SAMPLE_BLOCKS = tuple((r, r + 64) for r in (0, 544, 1056, 1568, 2016, 2048, 2592, 3104, 3616,
                                             4096, 4640, 5152, 6144, 6688, 7200, 7712, 8128))


def _gqa_rows_f64(torch, qn, K, V, gate, T, chunk=512, rel=2e-3):
    """Every row of a causal GQA prefill from position 0 in float64 on the
    GPU (a torch reference, for the all-rows sweep; the ordered oracle
    checks the sampled blocks): the reference's rounding points
    (c/attn.h:337-368, 524-531) -- A = rnd(rnd(q.k) * scale), P =
    rnd(e^{A-m} / sum e), o = rnd(sum P V), y = rnd(o * rnd(sigmoid(g)))
    -- with float64 sums in place of the ordered fp32 ones. Returns y codes
    [T, NH*D] and esc_y = |rnd(sigmoid(g))| * (sum_j P_j |V_jd| + the
    rounding-flip allowance of attn_util.attn_esc_rows: scores within the
    fp32 summation bound of a bf16 midpoint and probabilities within the
    exp / divide window of one may round the other way)."""
    dev = torch.device("cuda")

    def f64(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(
            torch.bfloat16).double()

    def rnd(x):
        return x.float().bfloat16().double()

    def mid(x):                      # distance to the nearest bf16 midpoint, and the ulp
        ax = x.abs()
        ulp = torch.exp2(torch.floor(torch.log2(ax.clamp_min(1e-300))) - 7)
        f = ax / ulp
        return (f - torch.floor(f) - 0.5).abs() * ulp, ulp

    grp = NH // NKV
    scale = 1.0 / 16.0
    q = f64(qn).reshape(T, NH, D)
    Kd, Vd = f64(K), f64(V)
    g = rnd(torch.sigmoid(f64(gate).reshape(T, NH, D)))
    y = torch.empty((T, NH, D), dtype=torch.float64, device=dev)
    esc = torch.empty_like(y)
    for r0 in range(0, T, chunk):
        r1 = min(T, r0 + chunk)
        pos = torch.arange(r0, r1, device=dev)
        keys = torch.arange(r1, device=dev)
        masked = keys[None, None, :] > pos[:, None, None]
        for hk in range(NKV):
            qh = q[r0:r1, hk * grp:(hk + 1) * grp]                      # [n, grp, D]
            Kh, Vh = Kd[:r1, hk], Vd[:r1, hk]
            Va = Vh.abs()
            s = torch.einsum("ngd,kd->ngk", qh, Kh)
            A = rnd(rnd(s) * scale).masked_fill(masked, float("-inf"))
            e = torch.exp(A - A.amax(2, keepdim=True))
            Pu = e / e.sum(2, keepdim=True)
            o = rnd(torch.einsum("ngk,kd->ngd", rnd(Pu), Vh))
            sl = slice(hk * grp, (hk + 1) * grp)
            y[r0:r1, sl] = rnd(o * g[r0:r1, sl])
            ee = torch.einsum("ngk,kd->ngd", Pu, Va)
            tabs = torch.einsum("ngd,kd->ngk", qh.abs(), Kh.abs())
            dist, ulp = mid(s)
            sflip = (dist <= 2.0 * D * 2.0 ** -24 * tabs) & ~masked
            dS = torch.where(sflip, Pu * torch.expm1(ulp * scale), torch.zeros_like(Pu))
            pd, pulp = mid(Pu)
            pflip = (pd <= 4e-6 * Pu) & ~masked
            dP = dS + torch.where(pflip, pulp, torch.zeros_like(Pu))
            allow = torch.einsum("ngk,kd->ngd", dP, Va) + dS.sum(2, keepdim=True) * ee
            esc[r0:r1, sl] = (ee + allow * (1.02 / rel)) * g[r0:r1, sl].abs()
    yc = y.float().bfloat16().view(torch.int16).cpu().numpy().view(np.uint16)
    return yc.reshape(T, NH * D), esc.cpu().numpy().reshape(T, NH * D)


@pytest.mark.timeout(400)
def test_config3_full_sampled(hip, orc):
    """T=8192 causal prefill from position 0. The whole
    cache fill bit-exact; outputs of all 16 heads on the sampled row
    blocks against the oracle's ordered GQA rows over keys 0..row."""
    import torch
    T = 8192
    rng = np.random.default_rng(24)
    w = synth.attn_weights(rng)
    tok = synth.attn_tokens(rng, T)
    print(f"[config3] T={T} sampled rows {SAMPLE_BLOCKS}", flush=True)
    layer = hip.attn_layer(synth.ATTN_DIMS, {n: _td(torch, a) for n, a in w.items()})
    t = {n: _td(torch, a) for n, a in tok.items()}
    dk = torch.zeros((1, NKV, T, D), dtype=torch.int16, device="cuda")
    dv = torch.zeros((1, NKV, T // 32, D, 32), dtype=torch.int16, device="cuda")
    y = torch.empty((T, NH * D), dtype=torch.int16, device="cuda")
    hip.attn_prefill(layer, [0, T], [0], t["qg"], t["k"], t["v"], dk, dv, T, y)
    torch.cuda.synchronize()
    yh = _h(y)
    kc = np.zeros(T * NKV * D, np.uint16)
    vc = np.zeros(T * NKV * D, np.uint16)
    cu = np.array([0, T], np.int32)
    pos0 = np.zeros(1, np.int32)
    qn = orc.attn_prep_off(synth.ATTN_DIMS, w, cu, pos0, tok["qg"], tok["k"], tok["v"], kc, vc,
                           np.zeros(1, np.int64), nthreads=NTHREADS)
    _check_appended(dk, dv, kc, vc, np.array([0, kc.size]), pos0, [T], T, hip)
    K = kc.reshape(T, NKV, D)
    V = vc.reshape(T, NKV, D)
    scale = np.float32(1.0 / 16.0)
    gate = tok["qg"].reshape(T, NH, 2 * D)[:, :, D:]
    for r0, r1 in SAMPLE_BLOCKS:
        n = r1 - r0
        ao = orc.attn_gqa_mt(np.ascontiguousarray(qn[r0:r1]), np.ascontiguousarray(K[:r1]),
                             np.ascontiguousarray(V[:r1]), n, r1, NH, NKV, D, scale,
                             nthreads=NTHREADS)
        y_o = orc.attn_outgate(ao, np.ascontiguousarray(gate[r0:r1]).reshape(-1))
        esc = attn_esc_rows(qn[r0:r1], K, V, np.arange(r0, r1), NH, NKV, D)
        st = assert_bf16_esc(yh[r0:r1], y_o.reshape(n, NH * D), esc, ulps=2,
                             what=f"config3 rows {r0}..{r1 - 1}")
        print(f"[config3] rows {r0}..{r1 - 1}: {st}", flush=True)
    # every row and head against the float64 torch reference (its sums in
    # another order than the reference's ascending fp32 ones: the same esc
    # tolerance class with the same rounding-flip allowance)
    y_t, esc_t = _gqa_rows_f64(torch, qn, K, V, gate, T)
    st = assert_bf16_esc(yh, y_t, esc_t, ulps=2, what="config3 all rows (float64 reference)")
    print(f"[config3] all {T} rows: {st}", flush=True)


def test_config4_full(hip, orc):
    """BASELINE config 4 on the benchmark's own draw: three GDN layers and
    one GQA layer over 128 sequences, back to back on the library stream,
    every layer against the oracle."""
    import torch
    ctx, k = synth.mixed_block_shape(128, 15)
    B = len(ctx)
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    T = int(cu[-1])
    rows = ctx + k
    max_seq = int(-(-int(rows.max()) // 32) * 32)
    print(f"[config4] B={B} T={T} ctx mean {ctx.mean():.0f} max {ctx.max()}", flush=True)
    rng = np.random.default_rng(25)
    g = torch.Generator(device="cuda").manual_seed(25)
    gd = synth.GDN_DIMS
    layers = []
    for _ in range(3):
        w = synth.gdn_weights(rng)
        tok = synth.gdn_tokens(rng, T)
        conv, S = synth.gdn_state(rng, B)
        L = dict(w=w, tok=tok, conv=conv, S=S)
        L["layer"] = hip.gdn_layer(gd, {n: _td(torch, a) for n, a in w.items()})
        L["t"] = {n: _td(torch, a) for n, a in tok.items()}
        L["dconv"] = _td(torch, conv)
        L["dS"] = torch.empty((B,) + S.shape[1:], dtype=torch.float32, device="cuda")
        hip.gdn_state_pack(_td(torch, S), L["dS"])
        L["y"] = torch.empty((T, gd[1] * gd[3]), dtype=torch.int16, device="cuda")
        layers.append(L)
    dk, dv, off, hk, hv = _fill_caches(hip, torch, g, B, ctx, rows, max_seq)
    aw = synth.attn_weights(rng)
    atok = synth.attn_tokens(rng, T)
    alayer = hip.attn_layer(synth.ATTN_DIMS, {n: _td(torch, a) for n, a in aw.items()})
    at = {n: _td(torch, a) for n, a in atok.items()}
    ay = torch.empty((T, NH * D), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()

    for L in layers:
        hip.gdn_decode(L["layer"], cu, L["t"]["qkv"], L["t"]["z"], L["t"]["a"], L["t"]["b"],
                       L["dconv"], L["dS"], L["y"])
    hip.attn_decode(alayer, cu, ctx, at["qg"], at["k"], at["v"], dk, dv, max_seq, ay)
    torch.cuda.synchronize()

    for i, L in enumerate(layers):
        c_o, S_o = L["conv"].copy(), L["S"].copy()
        tk = L["tok"]
        y_o = orc.gdn_mixer(gd, L["w"], cu, tk["qkv"], tk["z"], tk["a"], tk["b"], c_o, S_o,
                            nthreads=NTHREADS)
        st = assert_bf16_close(_h(L["y"]), y_o, what=f"config4 gdn{i} y")
        assert np.array_equal(_h(L["dconv"]), c_o), f"config4 gdn{i} conv state"
        S_ref = torch.empty_like(L["dS"])
        hip.gdn_state_unpack(L["dS"], S_ref)
        torch.cuda.synchronize()
        e = assert_state_close(S_ref.cpu().numpy(), S_o, what=f"config4 gdn{i} S")
        print(f"[config4] gdn{i} y {st} S rel {e:.3g}", flush=True)
        del L["dS"], S_ref

    y_o, qf, _, _ = orc.attn_mixer_off(synth.ATTN_DIMS, aw, cu, ctx, atok["qg"], atok["k"],
                                       atok["v"], hk, hv, off[:-1], nthreads=NTHREADS,
                                       capture=True)
    _check_appended(dk, dv, hk, hv, off, ctx, k, max_seq, hip)
    esc = np.concatenate([
        attn_esc_rows(qf[cu[s]:cu[s + 1]], hk[off[s]:off[s + 1]].reshape(-1, NKV, D),
                      hv[off[s]:off[s + 1]].reshape(-1, NKV, D),
                      ctx[s] + np.arange(k[s]), NH, NKV, D) for s in range(B)])
    st = assert_bf16_esc(_h(ay), y_o, esc, ulps=2, what="config4 attn y")
    print(f"[config4] attn y {st}", flush=True)


def test_gdn_decode_b500(hip, orc):
    """500 sequences of one token each: above the 480 sequences whose
    offsets travel by value, so the offsets go through device memory."""
    import torch
    rng = np.random.default_rng(26)
    B = 500
    gd = synth.GDN_DIMS
    w = synth.gdn_weights(rng)
    tok = synth.gdn_tokens(rng, B)
    conv, S = synth.gdn_state(rng, B)
    cu = np.arange(B + 1, dtype=np.int32)
    print(f"[gdn decode B=500]", flush=True)
    layer = hip.gdn_layer(gd, {n: _td(torch, a) for n, a in w.items()})
    t = {n: _td(torch, a) for n, a in tok.items()}
    dconv = _td(torch, conv)
    dS = torch.empty(S.shape, dtype=torch.float32, device="cuda")
    hip.gdn_state_pack(_td(torch, S), dS)
    y = torch.empty((B, gd[1] * gd[3]), dtype=torch.int16, device="cuda")
    hip.gdn_decode(layer, cu, t["qkv"], t["z"], t["a"], t["b"], dconv, dS, y)
    S_ref = torch.empty_like(dS)
    hip.gdn_state_unpack(dS, S_ref)
    torch.cuda.synchronize()
    c_o, S_o = conv.copy(), S.copy()
    y_o = orc.gdn_mixer(gd, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], c_o, S_o,
                        nthreads=NTHREADS)
    st = assert_bf16_close(_h(y), y_o, what="gdn decode B=500 y")
    assert np.array_equal(_h(dconv), c_o)
    e = assert_state_close(S_ref.cpu().numpy(), S_o, what="gdn decode B=500 S")
    print(f"[gdn decode B=500] y {st} S rel {e:.3g}", flush=True)
