"""GPU: the named-intermediate capture (apus_hip_trace_set, the hot-path
fields of the reference's ApusLayerTrace, c/layer.h:172-189) against the
oracle's captures of the same calls: the stage gates the reference runs on
its trace (tests/m4c) applied to the HIP mixers.

Bars: the conv+SiLU codes, beta codes, q/k after norm and RoPE and the
output gate codes are bit-exact; the decay g is fp32 within libm ulps
(relative 1e-6); rec_o of the fused decode within one bf16 ulp, of the
chunked prefill in its tolerance class (assert_bf16_rows); attno in the
attention class (esc); onorm equals the mixer output.
"""
import numpy as np
import pytest

import synth
from attn_util import attn_esc
from numerics import assert_bf16_close, assert_bf16_esc, assert_bf16_rows

pytestmark = pytest.mark.gpu


def _td(torch, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to("cuda")


def _h(t):
    return t.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("mode", ["decode", "prefill"])
def test_gdn_trace(hip, orc, mode):
    import torch
    rng = np.random.default_rng(51 if mode == "decode" else 52)
    gd = synth.GDN_DIMS
    hk, hv, dk, dv = gd
    cd = 2 * hk * dk + hv * dv
    lens = [1, 3, 4, 2] if mode == "decode" else [70, 5, 129]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    B, T = len(lens), int(cu[-1])
    w = synth.gdn_weights(rng)
    tok = synth.gdn_tokens(rng, T)
    conv, S = synth.gdn_state(rng, B, zero=(mode == "prefill"))
    layer = hip.gdn_layer(gd, {n: _td(torch, a) for n, a in w.items()})
    t = {n: _td(torch, a) for n, a in tok.items()}
    dconv = _td(torch, conv)
    dS = torch.empty(S.shape, dtype=torch.float32, device="cuda")
    hip.gdn_state_pack(_td(torch, S), dS)
    y = torch.empty((T, hv * dv), dtype=torch.int16, device="cuda")
    tr = dict(qkv_conv=torch.empty((T, cd), dtype=torch.int16, device="cuda"),
              beta=torch.empty((T, hv), dtype=torch.int16, device="cuda"),
              gdecay=torch.empty((T, hv), dtype=torch.float32, device="cuda"),
              rec_o=torch.empty((T, hv * dv), dtype=torch.int16, device="cuda"),
              onorm=torch.empty((T, hv * dv), dtype=torch.int16, device="cuda"))
    hip.trace_set(gdn=tr)
    try:
        f = hip.gdn_decode if mode == "decode" else hip.gdn_prefill
        f(layer, cu, t["qkv"], t["z"], t["a"], t["b"], dconv, dS, y)
        torch.cuda.synchronize()
    finally:
        hip.trace_set(None, None)
    c_o, S_o = conv.copy(), S.copy()
    y_o, trd = orc.gdn_mixer(gd, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], c_o, S_o,
                             trace=True)
    assert np.array_equal(_h(tr["qkv_conv"]), trd["qkv_conv"]), "qkv_conv"
    assert np.array_equal(_h(tr["beta"]), trd["beta"]), "beta"
    g = tr["gdecay"].cpu().numpy()
    assert np.allclose(g, trd["gdecay"], rtol=1e-6, atol=0), "gdecay"
    if mode == "decode":
        assert_bf16_close(_h(tr["rec_o"]), trd["rec_o"], what="rec_o")
    else:
        assert_bf16_rows(_h(tr["rec_o"]), trd["rec_o"], dv, what="rec_o")
    assert torch.equal(tr["onorm"], y), "onorm is the mixer output"


@pytest.mark.parametrize("mode", ["decode", "prefill"])
def test_attn_trace(hip, orc, mode):
    import torch
    rng = np.random.default_rng(53 if mode == "decode" else 54)
    dims = synth.ATTN_DIMS
    nh, nkv, d, rot, theta = dims
    lens = [1, 4, 2] if mode == "decode" else [37, 1, 70]
    pos0 = np.array([30, 100, 7] if mode == "decode" else [0, 12, 40], np.int32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    B, T = len(lens), int(cu[-1])
    ms = 128
    w = synth.attn_weights(rng)
    tok = synth.attn_tokens(rng, T)
    kc = synth.normal_bf16(rng, (B, ms, nkv, d))
    vc = synth.normal_bf16(rng, (B, ms, nkv, d))
    layer = hip.attn_layer(dims, {n: _td(torch, a) for n, a in w.items()})
    dk = torch.empty((B, nkv, ms, d), dtype=torch.int16, device="cuda")
    dv = torch.empty_like(dk)
    for s in range(B):
        hip.attn_cache_pack(_td(torch, kc[s]), _td(torch, vc[s]), ms, nkv, d, dk[s], dv[s], ms)
    t = {n: _td(torch, a) for n, a in tok.items()}
    y = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    tr = dict(qf=torch.empty((T, nh * d), dtype=torch.int16, device="cuda"),
              kf=torch.empty((T, nkv * d), dtype=torch.int16, device="cuda"),
              attno=torch.empty((T, nh * d), dtype=torch.int16, device="cuda"),
              mgate=torch.empty((T, nh * d), dtype=torch.int16, device="cuda"))
    hip.trace_set(attn=tr)
    try:
        f = hip.attn_decode if mode == "decode" else hip.attn_prefill
        f(layer, cu, pos0, t["qg"], t["k"], t["v"], dk, dv, ms, y)
        torch.cuda.synchronize()
    finally:
        hip.trace_set(None, None)
    k_o, v_o = kc.copy(), vc.copy()
    off = np.arange(B, dtype=np.int64) * ms * nkv * d
    y_o, qf, kf, ao = orc.attn_mixer_off(dims, w, cu, pos0, tok["qg"], tok["k"], tok["v"],
                                         k_o.reshape(-1), v_o.reshape(-1), off, capture=True)
    assert np.array_equal(_h(tr["qf"]), qf), "qf"
    assert np.array_equal(_h(tr["kf"]), kf), "kf"
    esc = attn_esc(qf, k_o, v_o, cu, pos0, nh, nkv, d)
    assert_bf16_esc(_h(tr["attno"]), ao, esc, ulps=1, what="attno")
    gate = np.ascontiguousarray(tok["qg"].reshape(T, nh, 2 * d)[:, :, d:]).reshape(-1)
    one = np.full(gate.shape, 0x3F80, np.uint16)              # rnd(1 * g) = g
    assert np.array_equal(_h(tr["mgate"]).reshape(-1), orc.attn_outgate(one, gate)), "mgate"
