"""GPU parity: BASELINE config 4's hybrid decode block -- three Gated
DeltaNet layers and one gated-GQA layer (the model's 3:1 ratio) -- on one
ragged batch in which every sequence verifies 1..4 tokens at a log-normal
cached context (contexts clipped small so the oracle stays fast).

The four mixers run back to back on the library's stream with no
synchronisation between them (as a model's decode step issues them), each
layer with its own weights, conv / recurrent state and KV cache, sharing
the batch metadata and the library's scratch. Every layer is then held to
its own tier's bar against the oracle: the GDN outputs within 1 bf16 ulp
and 2e-3 relative with the conv state bit-exact and the recurrent state
within 1e-4; the attention output in the esc tolerance class with the
appended cache rows bit-exact (tests/numerics.py).
"""
import numpy as np
import pytest

import synth
from attn_util import attn_esc
from numerics import assert_bf16_close, assert_bf16_esc, assert_state_close

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to("cuda")


def test_mixed_block_config4_shape(hip, orc):
    import torch
    rng = np.random.default_rng(40)
    B = 8
    ctx = synth.lognormal_contexts(rng, B, mu=np.log(300.0), lo=40, hi=700)
    k = rng.integers(1, 5, B).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    pos0 = ctx.astype(np.int32)
    T = int(cu[-1])
    print(f"[block] B={B} ctx={pos0.tolist()} k={k.tolist()}", flush=True)

    # three GDN layers
    gd = synth.GDN_DIMS
    layers = []
    for _ in range(3):
        w = synth.gdn_weights(rng)
        tok = synth.gdn_tokens(rng, T)
        conv, S = synth.gdn_state(rng, B)
        L = dict(w=w, tok=tok, conv=conv, S=S)
        L["layer"] = hip.gdn_layer(gd, {n: _dev(torch, v) for n, v in w.items()})
        L["t"] = {n: _dev(torch, v) for n, v in tok.items()}
        L["dconv"] = _dev(torch, conv)
        L["dS"] = torch.empty((B,) + S.shape[1:], dtype=torch.float32, device="cuda")
        hip.gdn_state_pack(_dev(torch, S), L["dS"])
        L["y"] = torch.empty((T, gd[1] * gd[3]), dtype=torch.int16, device="cuda")
        layers.append(L)

    # one gated-GQA layer
    ad = synth.ATTN_DIMS
    nh, nkv, d, rot, theta = ad
    max_seq = int(-(-int((pos0 + k).max()) // 32) * 32)
    aw = synth.attn_weights(rng)
    atok = synth.attn_tokens(rng, T)
    kc = synth.normal_bf16(rng, (B, max_seq, nkv, d))
    vc = synth.normal_bf16(rng, (B, max_seq, nkv, d))
    alayer = hip.attn_layer(ad, {n: _dev(torch, v) for n, v in aw.items()})
    dk = torch.empty((B, nkv, max_seq, d), dtype=torch.int16, device="cuda")
    dv = torch.empty((B, nkv, max_seq // 32, d, 32), dtype=torch.int16, device="cuda")
    for s in range(B):
        hip.attn_cache_pack(_dev(torch, kc[s]), _dev(torch, vc[s]), max_seq, nkv, d, dk[s], dv[s],
                            max_seq)
    at = {n: _dev(torch, v) for n, v in atok.items()}
    ay = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()

    # the block: four mixers back to back, one synchronisation at the end
    for L in layers:
        hip.gdn_decode(L["layer"], cu, L["t"]["qkv"], L["t"]["z"], L["t"]["a"], L["t"]["b"],
                       L["dconv"], L["dS"], L["y"])
    hip.attn_decode(alayer, cu, pos0, at["qg"], at["k"], at["v"], dk, dv, max_seq, ay)
    torch.cuda.synchronize()

    for i, L in enumerate(layers):
        c_o, S_o = L["conv"].copy(), L["S"].copy()
        t = L["tok"]
        y_o = orc.gdn_mixer(gd, L["w"], cu, t["qkv"], t["z"], t["a"], t["b"], c_o, S_o)
        st = assert_bf16_close(L["y"].cpu().numpy().view(np.uint16), y_o, what=f"block gdn{i} y")
        assert np.array_equal(L["dconv"].cpu().numpy().view(np.uint16), c_o), f"gdn{i} conv"
        S_ref = torch.empty((B,) + L["S"].shape[1:], dtype=torch.float32, device="cuda")
        hip.gdn_state_unpack(L["dS"], S_ref)
        torch.cuda.synchronize()
        e = assert_state_close(S_ref.cpu().numpy(), S_o, what=f"block gdn{i} S")
        print(f"[block] gdn{i} y {st} S rel {e:.3g}", flush=True)

    k_o, v_o = kc.copy(), vc.copy()
    y_o, qf, _ = orc.attn_mixer(ad, aw, cu, pos0, atok["qg"], atok["k"], atok["v"], k_o, v_o,
                                max_seq * nkv * d, capture=True)
    esc = attn_esc(qf, k_o, v_o, cu, pos0, nh, nkv, d)
    st = assert_bf16_esc(ay.cpu().numpy().view(np.uint16), y_o, esc, ulps=2, what="block attn y")
    rk = torch.empty((max_seq, nkv, d), dtype=torch.int16, device="cuda")
    rv = torch.empty_like(rk)
    for s in range(B):
        hip.attn_cache_unpack(dk[s], dv[s], max_seq, nkv, d, max_seq, rk, rv)
        torch.cuda.synchronize()
        assert np.array_equal(rk.cpu().numpy().view(np.uint16), k_o[s]), f"k cache seq {s}"
        assert np.array_equal(rv.cpu().numpy().view(np.uint16), v_o[s]), f"v cache seq {s}"
    print(f"[block] attn y {st}", flush=True)
