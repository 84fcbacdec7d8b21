"""GPU: the allocation-free chunked GDN prefill
(apus_hip_gdn_prefill_noalloc) against the allocating entry point
(apus_hip_gdn_prefill), called through the C ABI on the same inputs:
outputs, conv states and recurrent states bit-identical, on two calls in a
row -- the second smaller, so it runs in the scratch the first one left
behind -- and an oversize call refused with an error that names the size
it needs. (The allocating path is itself held to the oracle by
test_gpu_gdn_prefill.py.)"""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def _td(torch, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to("cuda")


def _case(hip, torch, rng, lens, layer):
    gd = synth.GDN_DIMS
    hk, hv, dk, dv = gd
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    B, T = len(lens), int(cu[-1])
    tok = synth.gdn_tokens(rng, T)
    conv, S = synth.gdn_state(rng, B)
    t = {n: _td(torch, a) for n, a in tok.items()}
    outs = []
    for f in (hip.gdn_prefill, hip.gdn_prefill_noalloc):
        dconv = _td(torch, conv)
        dS = torch.empty(S.shape, dtype=torch.float32, device="cuda")
        hip.gdn_state_pack(_td(torch, S), dS)
        y = torch.empty((T, hv * dv), dtype=torch.int16, device="cuda")
        f(layer, cu, t["qkv"], t["z"], t["a"], t["b"], dconv, dS, y)
        outs.append((y, dconv, dS))
    torch.cuda.synchronize()
    for name, x, z in zip(("y", "conv state", "S"), outs[0], outs[1]):
        assert torch.equal(x, z), f"{name} differs for lengths {lens}"


def test_noalloc_prefill_matches(hip):
    import torch
    rng = np.random.default_rng(61)
    w = synth.gdn_weights(rng)
    layer = hip.gdn_layer(synth.GDN_DIMS, {n: _td(torch, a) for n, a in w.items()})
    print("[noalloc] 3 sequences (600, 130, 1 tokens), then 2 (100, 37)", flush=True)
    _case(hip, torch, rng, [600, 130, 1], layer)
    _case(hip, torch, rng, [100, 37], layer)


def test_noalloc_prefill_rejects_oversize(hip):
    import torch
    rng = np.random.default_rng(62)
    gd = synth.GDN_DIMS
    hk, hv, dk, dv = gd
    w = synth.gdn_weights(rng)
    layer = hip.gdn_layer(gd, {n: _td(torch, a) for n, a in w.items()})
    T = 4096
    cd = 2 * hk * dk + hv * dv
    qkv = torch.zeros((T, cd), dtype=torch.int16, device="cuda")
    z = torch.zeros((T, hv * dv), dtype=torch.int16, device="cuda")
    ab = torch.zeros((T, hv), dtype=torch.int16, device="cuda")
    conv = torch.zeros((1, cd * 3), dtype=torch.int16, device="cuda")
    S = torch.zeros((1, hv, dk, dv), dtype=torch.float32, device="cuda")
    y = torch.empty((T, hv * dv), dtype=torch.int16, device="cuda")
    with pytest.raises(hip.ApusHipError) as e:
        hip.gdn_prefill_noalloc(layer, [0, T], qkv, z, ab, ab, conv, S, y)
    assert e.value.code == 1 and "needs" in str(e.value)
