"""GPU parity: one layer's mixer WITH its projections (c/layer.h:236-331),
apus_hip_gdn_layer_decode[_slots] and apus_hip_attn_layer_decode[_paged]:
ln1 -> one fused input-projection launch -> mixer -> output projection.

Checked in three ways, each stage against the oracle (whose bf16 GEMM and
mixers are pinned bitwise to the reference's own c/bf16.h / c/gdn.h /
c/attn.h in the CPU tests):
  * the fused call equals, bit for bit, the same layer composed of the
    separate entry points (four / three MFMA GEMMs, the mixer, the output
    GEMM) -- the segmented launch computes every element in the same order;
  * each input projection of that composition is within the MFMA GEMM's
    tolerance class of orc.bf16_gemm (|c - r| <= 2e-3 (|r| + esc));
  * the mixer on those projections is held to its own bar against the
    oracle mixer on the same (downloaded) projections, and the output GEMM
    to the GEMM class against orc.bf16_gemm of the mixer output.
Slot-mapped / paged forms equal the flat forms bitwise.
"""
import numpy as np
import pytest

import synth
from attn_util import attn_esc
from numerics import assert_bf16_close, assert_bf16_esc, assert_state_close

pytestmark = pytest.mark.gpu

H = 2048


def _dev(torch, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to("cuda")


def _h(t):
    return t.cpu().numpy().view(np.uint16)


def _gemm_class(c, w, x, orc, what):
    """c [M, O] codes against orc.bf16_gemm(w, x) in the MFMA class."""
    r = orc.bf16_gemm(w, x)
    cf = synth.bf16_f32(c).astype(np.float64)
    rf = synth.bf16_f32(r).astype(np.float64)
    esc = np.abs(synth.bf16_f32(x).astype(np.float64)) @ np.abs(synth.bf16_f32(w).astype(np.float64)).T
    assert np.all(np.abs(cf - rf) <= 2e-3 * (np.abs(rf) + esc)), what
    nrm = np.linalg.norm(cf - rf) / np.linalg.norm(rf)
    assert nrm <= 2e-3, (what, nrm)
    return float(nrm)


def _gdn_proj_weights(rng, dims):
    hk, hv, dk, dv = dims
    cd, vd = 2 * hk * dk + hv * dv, hv * dv
    s = H ** -0.5
    return dict(w_qkv=synth.normal_bf16(rng, (cd, H), s), w_z=synth.normal_bf16(rng, (vd, H), s),
                w_b=synth.normal_bf16(rng, (hv, H), s), w_a=synth.normal_bf16(rng, (hv, H), s),
                w_out=synth.normal_bf16(rng, (H, vd), vd ** -0.5))


def test_gdn_layer_decode(hip, orc):
    import torch
    rng = np.random.default_rng(71)
    dims = synth.GDN_DIMS
    hk, hv, dk, dv = dims
    cd, vd = 2 * hk * dk + hv * dv, hv * dv
    k = np.array([1, 3, 2, 4, 1], np.int32)
    B, cu = len(k), np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    T = int(cu[-1])
    print(f"[layer gdn] B={B} k={k.tolist()}", flush=True)
    w = synth.gdn_weights(rng)
    pw = _gdn_proj_weights(rng, dims)
    ln1 = synth.normal_bf16(rng, (T, H))
    conv, S = synth.gdn_state(rng, B)
    layer = hip.gdn_layer(dims, {n: _dev(torch, v) for n, v in w.items()})
    proj = hip.gdn_proj(H, {n: _dev(torch, v) for n, v in pw.items()})
    dln = _dev(torch, ln1)

    def states():
        dS = torch.empty((B,) + S.shape[1:], dtype=torch.float32, device="cuda")
        hip.gdn_state_pack(_dev(torch, S), dS)
        return _dev(torch, conv), dS

    # fused
    c1, S1 = states()
    ao1 = torch.empty((T, H), dtype=torch.int16, device="cuda")
    hip.gdn_layer_decode(layer, proj, cu, dln, c1, S1, ao1)
    # composed of the separate entry points
    c2, S2 = states()
    P = proj._tensors
    qkv = torch.empty((T, cd), dtype=torch.int16, device="cuda")
    z = torch.empty((T, vd), dtype=torch.int16, device="cuda")
    a = torch.empty((T, hv), dtype=torch.int16, device="cuda")
    b = torch.empty((T, hv), dtype=torch.int16, device="cuda")
    for wt, out in ((P["w_qkv"], qkv), (P["w_z"], z), (P["w_b"], b), (P["w_a"], a)):
        hip.bf16_gemm_dev(wt, dln, out, exact=False)
    y = torch.empty((T, vd), dtype=torch.int16, device="cuda")
    hip.gdn_decode(layer, cu, qkv, z, a, b, c2, S2, y)
    ao2 = torch.empty((T, H), dtype=torch.int16, device="cuda")
    hip.bf16_gemm_dev(P["w_out"], y, ao2, exact=False)
    # slot-mapped (shuffled slots of a larger pool)
    nsl = B + 3
    perm = rng.permutation(nsl)[:B].astype(np.int32)
    cpool = torch.zeros((nsl, cd * 3), dtype=torch.int16, device="cuda")
    Spool = torch.zeros((nsl,) + S.shape[1:], dtype=torch.float32, device="cuda")
    c0, S0 = states()
    for s in range(B):
        cpool[perm[s]] = c0[s]
        Spool[perm[s]] = S0[s]
    ao3 = torch.empty((T, H), dtype=torch.int16, device="cuda")
    hip.gdn_layer_decode_slots(layer, proj, perm, perm, cu, dln, cpool.data_ptr(),
                               Spool.data_ptr(), ao3)
    torch.cuda.synchronize()

    assert np.array_equal(_h(ao1), _h(ao2)), "fused layer != separate launches"
    assert np.array_equal(_h(c1), _h(c2)) and torch.equal(S1, S2)
    assert np.array_equal(_h(ao3), _h(ao1)), "slotted layer != flat layer"
    for s in range(B):
        assert torch.equal(cpool[perm[s]], c1[s]) and torch.equal(Spool[perm[s]], S1[s])

    # stage by stage against the oracle
    proj_h = dict(qkv=_h(qkv), z=_h(z), a=_h(a), b=_h(b))
    for name, wn in (("qkv", "w_qkv"), ("z", "w_z"), ("a", "w_a"), ("b", "w_b")):
        nrm = _gemm_class(proj_h[name], pw[wn], ln1, orc, f"in_proj {name}")
        print(f"[layer gdn] {name} normwise {nrm:.3g}", flush=True)
    c_o, S_o = conv.copy(), S.copy()
    y_o = orc.gdn_mixer(dims, w, cu, proj_h["qkv"], proj_h["z"], proj_h["a"], proj_h["b"], c_o, S_o)
    st = assert_bf16_close(_h(y), y_o, what="layer gdn mixer y")
    assert np.array_equal(_h(c1), c_o), "conv state"
    S_ref = torch.empty((B,) + S.shape[1:], dtype=torch.float32, device="cuda")
    hip.gdn_state_unpack(S1, S_ref)
    torch.cuda.synchronize()
    e = assert_state_close(S_ref.cpu().numpy(), S_o, what="layer gdn S")
    nrm = _gemm_class(_h(ao1), pw["w_out"], _h(y), orc, "w_out")
    print(f"[layer gdn] mixer {st} S rel {e:.3g}; w_out normwise {nrm:.3g}", flush=True)


def test_attn_layer_decode(hip, orc):
    import torch
    rng = np.random.default_rng(72)
    dims = synth.ATTN_DIMS
    nh, nkv, d, rot, theta = dims
    k = np.array([1, 4, 2], np.int32)
    B, cu = len(k), np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    pos0 = np.array([37, 300, 5], np.int32)
    T = int(cu[-1])
    max_seq = 320
    print(f"[layer attn] B={B} k={k.tolist()} pos0={pos0.tolist()}", flush=True)
    w = synth.attn_weights(rng)
    s = H ** -0.5
    pw = dict(wq=synth.normal_bf16(rng, (nh * 2 * d, H), s),
              wk=synth.normal_bf16(rng, (nkv * d, H), s),
              wv=synth.normal_bf16(rng, (nkv * d, H), s),
              wo=synth.normal_bf16(rng, (H, nh * d), (nh * d) ** -0.5))
    ln1 = synth.normal_bf16(rng, (T, H))
    kc = synth.normal_bf16(rng, (B, max_seq, nkv, d))
    vc = synth.normal_bf16(rng, (B, max_seq, nkv, d))
    layer = hip.attn_layer(dims, {n: _dev(torch, v) for n, v in w.items()})
    proj = hip.attn_proj(H, {n: _dev(torch, v) for n, v in pw.items()})
    dln = _dev(torch, ln1)

    def caches():
        dk = torch.empty((B, nkv, max_seq, d), dtype=torch.int16, device="cuda")
        dv = torch.empty((B, nkv, max_seq // 32, d, 32), dtype=torch.int16, device="cuda")
        for q in range(B):
            hip.attn_cache_pack(_dev(torch, kc[q]), _dev(torch, vc[q]), max_seq, nkv, d, dk[q],
                                dv[q], max_seq)
        return dk, dv

    dk1, dv1 = caches()
    ao1 = torch.empty((T, H), dtype=torch.int16, device="cuda")
    hip.attn_layer_decode(layer, proj, cu, pos0, dln, dk1, dv1, max_seq, ao1)
    dk2, dv2 = caches()
    P = proj._tensors
    qg = torch.empty((T, nh * 2 * d), dtype=torch.int16, device="cuda")
    kk = torch.empty((T, nkv * d), dtype=torch.int16, device="cuda")
    vv = torch.empty((T, nkv * d), dtype=torch.int16, device="cuda")
    for wt, out in ((P["wq"], qg), (P["wk"], kk), (P["wv"], vv)):
        hip.bf16_gemm_dev(wt, dln, out, exact=False)
    y = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    hip.attn_decode(layer, cu, pos0, qg, kk, vv, dk2, dv2, max_seq, y)
    ao2 = torch.empty((T, H), dtype=torch.int16, device="cuda")
    hip.bf16_gemm_dev(P["wo"], y, ao2, exact=False)
    # paged: each sequence's blocks from a pool, in shuffled rows
    pool = hip.KvPool(1, nkv, d, B * (max_seq // 32) + 4, B + 2, max_seq // 32)
    rows = []
    for q in range(B):
        rows.append(pool.open())
        pool.reserve(rows[-1], max_seq)
    kv = pool.cache(0)
    for q in range(B):
        hip.attn_cache_pack_paged(_dev(torch, kc[q]), _dev(torch, vc[q]), max_seq, nkv, d, kv,
                                  rows[q])
    ao3 = torch.empty((T, H), dtype=torch.int16, device="cuda")
    hip.attn_layer_decode_paged(layer, proj, rows, cu, pos0, dln, kv, ao3)
    torch.cuda.synchronize()
    assert np.array_equal(_h(ao1), _h(ao2)), "fused layer != separate launches"
    assert torch.equal(dk1, dk2) and torch.equal(dv1, dv2)
    assert np.array_equal(_h(ao3), _h(ao1)), "paged layer != flat layer"

    ph = dict(qg=_h(qg), k=_h(kk), v=_h(vv))
    for name, wn in (("qg", "wq"), ("k", "wk"), ("v", "wv")):
        nrm = _gemm_class(ph[name], pw[wn], ln1, orc, f"in_proj {name}")
        print(f"[layer attn] {name} normwise {nrm:.3g}", flush=True)
    k_o, v_o = kc.copy(), vc.copy()
    y_o, qf, _ = orc.attn_mixer(dims, w, cu, pos0, ph["qg"], ph["k"], ph["v"], k_o, v_o,
                                max_seq * nkv * d, capture=True)
    esc = attn_esc(qf, k_o, v_o, cu, pos0, nh, nkv, d)
    st = assert_bf16_esc(_h(y), y_o, esc, ulps=2, what="layer attn mixer y")
    nrm = _gemm_class(_h(ao1), pw["wo"], _h(y), orc, "wo")
    print(f"[layer attn] mixer {st}; wo normwise {nrm:.3g}", flush=True)
    pool.destroy()
