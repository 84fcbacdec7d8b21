"""GPU parity: chunked GDN prefill (apus_hip_gdn_prefill) against the
oracle's sequential recurrence.

The chunk (WY/UT) form sums in a different order from the reference's
token loop (c/gdn.h:627-635), so it is a tolerance class of it:
  * recurrent state: max |S - S_ref| / max |S_ref| <= 1e-4;
  * y (after rnd(o) and the three-rounding gated RMSNorm): normwise
    relative error <= 2e-3 and at most 4 bf16 ulps per element (an fp32
    ulp of o that crosses a bf16 rounding boundary moves rnd(o) by one
    ulp and each of the norm's three roundings by at most one more),
    elements small through cancellation judged against their row's rms
    (numerics.assert_bf16_rows);
  * conv state: bit-exact (pure copies of input codes).
Cases: ragged batches with partial chunks (1, 63, 64, 65, 130 tokens) from
a prior state, BASELINE config 1 (T=4096 from zero state), and a strong
decay case where cumulative in-chunk decay underflows fp32.
"""
import numpy as np
import pytest

import synth
from numerics import assert_bf16_close, assert_bf16_rows, assert_state_close

pytestmark = pytest.mark.gpu


def _dev(torch, arr):
    return torch.from_numpy(arr.view(np.int16) if arr.dtype == np.uint16 else arr).to("cuda")


def _run_prefill(hip, orc, rng, cu, zero_state=False, a_scale=1.0, tag=""):
    import torch
    dims = synth.GDN_DIMS
    B = len(cu) - 1
    T = int(cu[-1])
    w = synth.gdn_weights(rng)
    tok = synth.gdn_tokens(rng, T)
    if a_scale != 1.0:
        tok["a"] = synth.bf16_bits(synth.bf16_f32(tok["a"]) * np.float32(a_scale) + np.float32(4.0))
    conv, S = synth.gdn_state(rng, B, zero=zero_state)
    print(f"[gdn_prefill {tag}] B={B} T={T} cu={list(cu)[:8]}...", flush=True)
    c_o, S_o = conv.copy(), S.copy()
    y_o = orc.gdn_mixer(dims, w, np.asarray(cu, np.int32), tok["qkv"], tok["z"], tok["a"],
                        tok["b"], c_o, S_o)
    tw = {k: _dev(torch, v) for k, v in w.items()}
    layer = hip.gdn_layer(dims, tw)
    t = {k: _dev(torch, v) for k, v in tok.items()}
    dconv = _dev(torch, conv)
    dS_ref = torch.from_numpy(S).cuda()
    dS = torch.empty_like(dS_ref)
    hip.gdn_state_pack(dS_ref, dS)
    y = torch.empty((T, dims[1] * dims[3]), dtype=torch.int16, device="cuda")
    hip.gdn_prefill(layer, cu, t["qkv"], t["z"], t["a"], t["b"], dconv, dS, y)
    hip.gdn_state_unpack(dS, dS_ref)
    torch.cuda.synchronize()
    y_h = y.cpu().numpy().view(np.uint16)
    assert np.array_equal(dconv.cpu().numpy().view(np.uint16), c_o), "conv state"
    e = assert_state_close(dS_ref.cpu().numpy(), S_o, what=f"prefill S {tag}")
    st = assert_bf16_rows(y_h, y_o, 128, what=f"prefill y {tag}")
    print(f"[gdn_prefill {tag}] y {st} state rel {e:.3g}", flush=True)
    return st, e


def test_prefill_ragged(hip, orc):
    """Partial and exact chunks, a one-token sequence, prior state."""
    lens = [1, 63, 64, 65, 130, 7]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _run_prefill(hip, orc, np.random.default_rng(1001), cu, tag="ragged")


def test_prefill_config1(hip, orc):
    """batch 1, T=4096, zero initial state."""
    _run_prefill(hip, orc, np.random.default_rng(12), np.array([0, 4096], np.int32),
                 zero_state=True, tag="config1")


def test_prefill_strong_decay(hip, orc):
    """a shifted up by 4 (softplus ~ 4-8 per token, with A_log up to 2.7 the
    log decay reaches -100 per token): exp(gamma) of a chunk underflows and
    the state forgets within a few tokens."""
    _run_prefill(hip, orc, np.random.default_rng(77), np.array([0, 200], np.int32),
                 a_scale=2.0, tag="strong_decay")


def test_prefill_then_decode(hip, orc):
    """Prefill a prompt then decode one token from the device state: the
    state layout and conv state the prefill leaves are what decode reads."""
    import torch
    dims = synth.GDN_DIMS
    rng = np.random.default_rng(31)
    T = 100
    w = synth.gdn_weights(rng)
    tok = synth.gdn_tokens(rng, T + 1)
    conv, S = synth.gdn_state(rng, 1, zero=True)
    c_o, S_o = conv.copy(), S.copy()
    y_o = orc.gdn_mixer(dims, w, np.array([0, T + 1], np.int32), tok["qkv"], tok["z"], tok["a"],
                        tok["b"], c_o, S_o)
    tw = {k: _dev(torch, v) for k, v in w.items()}
    layer = hip.gdn_layer(dims, tw)
    t = {k: _dev(torch, v) for k, v in tok.items()}
    dconv = _dev(torch, conv)
    dS = torch.zeros(S.shape, dtype=torch.float32, device="cuda")
    y = torch.empty((T + 1, dims[1] * dims[3]), dtype=torch.int16, device="cuda")
    hip.gdn_prefill(layer, [0, T], t["qkv"][:T], t["z"][:T], t["a"][:T], t["b"][:T], dconv, dS,
                    y[:T])
    hip.gdn_decode(layer, [0, 1], t["qkv"][T:], t["z"][T:], t["a"][T:], t["b"][T:], dconv, dS,
                   y[T:])
    Su = torch.empty_like(dS)
    hip.gdn_state_unpack(dS, Su)
    torch.cuda.synchronize()
    assert np.array_equal(dconv.cpu().numpy().view(np.uint16), c_o)
    assert_state_close(Su.cpu().numpy(), S_o, what="prefill+decode S")
    assert_bf16_rows(y.cpu().numpy().view(np.uint16), y_o, 128, what="prefill+decode y")


@pytest.mark.parametrize("B", [260, 410])
def test_prefill_many_sequences(hip, orc, B):
    """Batches past the by-value metadata limits (256 sequences for the
    token-parallel kernels, 400 for the chunk kernels): the offsets then
    travel through a device copy."""
    rng = np.random.default_rng(B)
    lens = rng.integers(1, 5, B)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _run_prefill(hip, orc, rng, cu, tag=f"B{B}")


def test_prefill_batched_equals_alone(hip):
    """The reference's batch invariance (batched prefill == sequential,
    bitwise; tests/m9c): a ragged batch of 5 sequences and each sequence
    prefilled alone give the same outputs, conv state and recurrent state,
    bit for bit (a sequence's chunks start at its own first token either
    way)."""
    import torch
    rng = np.random.default_rng(95)
    dims = synth.GDN_DIMS
    k = [1, 63, 64, 65, 130]
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    B, T = len(k), int(cu[-1])
    w = synth.gdn_weights(rng)
    tok = synth.gdn_tokens(rng, T)
    conv, S = synth.gdn_state(rng, B)
    layer = hip.gdn_layer(dims, {n: _dev(torch, v) for n, v in w.items()})
    t = {n: _dev(torch, v) for n, v in tok.items()}
    dS0 = torch.empty((B,) + S.shape[1:], dtype=torch.float32, device="cuda")
    hip.gdn_state_pack(torch.from_numpy(S).cuda(), dS0)
    vd = dims[1] * dims[3]
    c1, S1 = _dev(torch, conv), dS0.clone()
    y1 = torch.empty((T, vd), dtype=torch.int16, device="cuda")
    hip.gdn_prefill(layer, cu, t["qkv"], t["z"], t["a"], t["b"], c1, S1, y1)
    c2, S2 = _dev(torch, conv), dS0.clone()
    y2 = torch.empty((T, vd), dtype=torch.int16, device="cuda")
    for s in range(B):
        a, b = int(cu[s]), int(cu[s + 1])
        hip.gdn_prefill(layer, [0, b - a], t["qkv"][a:b], t["z"][a:b], t["a"][a:b], t["b"][a:b],
                        c2[s:s + 1], S2[s:s + 1], y2[a:b])
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "outputs"
    assert torch.equal(c1, c2), "conv state"
    assert torch.equal(S1, S2), "recurrent state"
