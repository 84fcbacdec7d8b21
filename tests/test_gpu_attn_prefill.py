"""GPU parity: the gated-GQA causal prefill (apus_hip_attn_prefill) against
the oracle's mixer (c/layer.h wiring, token by token: append, then attend
positions 0..pos) on identical inputs.

Tolerance class: the kernel forms the reference's own probabilities
P = rnd(e^{A-m} / s) (c/attn.h:354-360) but sums q.k and P.V on MFMA in
another order. Every element is held to |c - r| <= 2e-3 (|r| + esc),
esc = sum_j P_j |V_jd| (the reference's esc form), or to 2 bf16 ulps (one
of rnd(o), carried through the gate's rnd(o * g)), and the tensor to 2e-3
normwise. The cache
rows the prefill appends (normed, roped k; raw v) must be bit-exact.
Cases: ragged batches with prior cache content and tile edges (16-token
query tiles, 32-key tiles), a longer causal run from position 0, and at
BASELINE config 3's full T=8192 a consistency property against the
decode kernel for the last tokens.
"""
import numpy as np
import pytest

import synth
from attn_util import attn_esc
from numerics import assert_bf16_esc

pytestmark = pytest.mark.gpu


def _td(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda")


def _run(hip, orc, rng, cu, pos0, max_seq, tag="", edit=None, dims=synth.ATTN_DIMS):
    import torch
    nh, nkv, d, rot, theta = dims
    B = len(cu) - 1
    T = int(cu[-1])
    print(f"[attn_prefill {tag}] B={B} T={T} pos0={list(pos0)[:6]} max_seq={max_seq}", flush=True)
    w = synth.attn_weights(rng, dims)
    tok = synth.attn_tokens(rng, T, dims)
    kc = synth.normal_bf16(rng, (B, max_seq, nkv, d))
    vc = synth.normal_bf16(rng, (B, max_seq, nkv, d))
    if edit:
        edit(tok, kc)
    k_o, v_o = kc.copy(), vc.copy()
    y_o, qf, _ = orc.attn_mixer(dims, w, np.asarray(cu, np.int32), np.asarray(pos0, np.int32),
                                tok["qg"], tok["k"], tok["v"], k_o, v_o, max_seq * nkv * d,
                                capture=True)
    esc = attn_esc(qf, k_o, v_o, np.asarray(cu), np.asarray(pos0), nh, nkv, d)
    layer = hip.attn_layer(dims, {k: _td(torch, v) for k, v in w.items()})
    dk = torch.empty((B, nkv, max_seq, d), dtype=torch.int16, device="cuda")
    dv = torch.empty((B, nkv, max_seq // 32, d, 32), dtype=torch.int16, device="cuda")
    for s in range(B):
        hip.attn_cache_pack(_td(torch, kc[s]), _td(torch, vc[s]), max_seq, nkv, d, dk[s], dv[s],
                            max_seq)
    y = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    t = {k: _td(torch, v) for k, v in tok.items()}
    hip.attn_prefill(layer, cu, pos0, t["qg"], t["k"], t["v"], dk, dv, max_seq, y)
    rk = torch.empty((max_seq, nkv, d), dtype=torch.int16, device="cuda")
    rv = torch.empty_like(rk)
    for s in range(B):
        hip.attn_cache_unpack(dk[s], dv[s], max_seq, nkv, d, max_seq, rk, rv)
        torch.cuda.synchronize()
        assert np.array_equal(rk.cpu().numpy().view(np.uint16), k_o[s]), f"k cache seq {s}"
        assert np.array_equal(rv.cpu().numpy().view(np.uint16), v_o[s]), f"v cache seq {s}"
    st = assert_bf16_esc(y.cpu().numpy().view(np.uint16), y_o, esc, ulps=2,
                         what=f"attn_prefill y {tag}")
    print(f"[attn_prefill {tag}] {st}", flush=True)
    return st


def test_prefill_small(hip, orc):
    """Two sequences: 37 tokens from position 0, 20 tokens after 50 cached."""
    _run(hip, orc, np.random.default_rng(11), [0, 37, 57], [0, 50], 128, tag="small")


def test_prefill_score_growth(hip, orc):
    """Scores that rise far above the first key step's: pass 1 takes its
    sums against a reference point that it raises only when a sum would
    leave the fp32 range, and this case makes every row raise it. Every q
    row is all ones (after the (1+w) norm all its unrotated dims have one
    sign) and the cached keys 0..31 are all -250, so their scores lie near
    -2,000 while the later keys' scores are O(1): ~2,000 above the first
    step's max, past the ~1,100 at which the sum against it would
    overflow. The reference's terms for keys 0..31 underflow to 0 as the
    kernel's do."""
    def edit(tok, kc):
        tok["qg"][:, :, :synth.ATTN_DIMS[2]] = synth.bf16_bits(np.float32(1.0))
        kc[:, :32] = synth.bf16_bits(np.float32(-250.0))
    _run(hip, orc, np.random.default_rng(14), [0, 40, 75], [64, 96], 192, tag="growth",
         edit=edit)


def test_prefill_long_prefix(hip, orc):
    """A continuation after a 30,000-position cached prefix: RoPE at large
    positions in the flash kernel's own q rows, and ~470 key tiles per
    query tile with the query rows at their end."""
    _run(hip, orc, np.random.default_rng(16), [0, 20], [30000], 30048, tag="long-prefix")


def test_prefill_one_kv_head(hip, orc):
    """One kv head (8 q heads): the prep kernel then keeps forming the q rows
    too (its k-row blocks would span more tokens than their metadata
    holds), while the flash kernel forms its own."""
    nh, nkv, d, rot, theta = synth.ATTN_DIMS
    _run(hip, orc, np.random.default_rng(15), [0, 45, 80], [0, 70], 160, tag="nkv1",
         dims=(8, 1, d, rot, theta))


def test_prefill_tile_edges(hip, orc):
    """Query counts around the 16-token tile (16, 17, 31, 32, 33, 1) and
    cached prefixes around the 32-key tile."""
    lens = [16, 17, 31, 32, 33, 1]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _run(hip, orc, np.random.default_rng(12), cu, [0, 31, 32, 63, 5, 100], 160, tag="edges")


def test_prefill_long(hip, orc):
    """One 2048-token causal prefill from position 0 (config 3's shape at a
    quarter of its length)."""
    _run(hip, orc, np.random.default_rng(13), [0, 2048], [0], 2048, tag="long")


def test_prefill_config3_vs_decode(hip):
    """BASELINE config 3 (T=8192 from position 0): the last 4 rows of the
    prefill equal, within the tolerance class, what the split-K decode
    kernel computes for those 4 tokens over the cache the prefill filled
    (the decode appends the same rows again, bit-identically)."""
    import torch
    dims = synth.ATTN_DIMS
    nh, nkv, d, rot, theta = dims
    T = 8192
    rng = np.random.default_rng(14)
    w = synth.attn_weights(rng)
    tok = synth.attn_tokens(rng, T)
    layer = hip.attn_layer(dims, {k: _td(torch, v) for k, v in w.items()})
    dk = torch.zeros((1, nkv, T, d), dtype=torch.int16, device="cuda")
    dv = torch.zeros((1, nkv, T // 32, d, 32), dtype=torch.int16, device="cuda")
    t = {k: _td(torch, v) for k, v in tok.items()}
    y = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    hip.attn_prefill(layer, [0, T], [0], t["qg"], t["k"], t["v"], dk, dv, T, y)
    dk2, dv2 = dk.clone(), dv.clone()
    y2 = torch.empty((4, nh * d), dtype=torch.int16, device="cuda")
    hip.attn_decode(layer, [0, 4], [T - 4], t["qg"][T - 4:], t["k"][T - 4:], t["v"][T - 4:],
                    dk2, dv2, T, y2)
    torch.cuda.synchronize()
    assert torch.equal(dk, dk2) and torch.equal(dv, dv2)
    a = y[T - 4:].cpu().numpy().view(np.uint16)
    b = y2.cpu().numpy().view(np.uint16)
    # both sides are tolerance-class results; the term scale of these rows
    # is taken as the mean output magnitude
    mag = np.abs(synth.bf16_f32(b).astype(np.float64)).mean()
    st = assert_bf16_esc(a, b, np.full(a.shape, mag), ulps=2,
                         what="config3 prefill vs decode")
    print(f"[attn_prefill config3] last rows vs decode {st}", flush=True)


@pytest.mark.parametrize("T,cut", [(12, 7), (300, 173), (1000, 513)])
def test_prefill_split_equals_oneshot(hip, T, cut):
    """The reference's chunking invariance (its one-shot T=12 prefill must
    equal a 7 + 5 chunking bitwise, tests/m4c/README.md): T tokens
    prefilled in one call and the same tokens in two calls (the second
    starting at position `cut` over the cache the first filled) give the
    same outputs and the same cache, bit for bit. A row's scores, its
    running max / sum and its P.V run over keys 0..pos in the same 32-key
    steps whichever call holds it."""
    import torch
    dims = synth.ATTN_DIMS
    nh, nkv, d, rot, theta = dims
    rng = np.random.default_rng(T)
    w = synth.attn_weights(rng)
    tok = synth.attn_tokens(rng, T)
    layer = hip.attn_layer(dims, {k: _td(torch, v) for k, v in w.items()})
    max_seq = -(-T // 32) * 32
    t = {k: _td(torch, v) for k, v in tok.items()}

    def fresh():
        return (torch.zeros((1, nkv, max_seq, d), dtype=torch.int16, device="cuda"),
                torch.zeros((1, nkv, max_seq // 32, d, 32), dtype=torch.int16, device="cuda"))

    dk1, dv1 = fresh()
    y1 = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    hip.attn_prefill(layer, [0, T], [0], t["qg"], t["k"], t["v"], dk1, dv1, max_seq, y1)
    dk2, dv2 = fresh()
    y2 = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    hip.attn_prefill(layer, [0, cut], [0], t["qg"][:cut], t["k"][:cut], t["v"][:cut], dk2, dv2,
                     max_seq, y2[:cut])
    hip.attn_prefill(layer, [0, T - cut], [cut], t["qg"][cut:], t["k"][cut:], t["v"][cut:],
                     dk2, dv2, max_seq, y2[cut:])
    torch.cuda.synchronize()
    assert torch.equal(dk1, dk2) and torch.equal(dv1, dv2), "cache"
    assert torch.equal(y1, y2), "outputs"


def test_prefill_batched_equals_alone(hip):
    """The reference's batch invariance (batched prefill == sequential,
    bitwise; tests/m9c): a ragged batch with cached prefixes and each
    sequence prefilled alone over its own cache give the same outputs and
    caches, bit for bit."""
    import torch
    dims = synth.ATTN_DIMS
    nh, nkv, d, rot, theta = dims
    rng = np.random.default_rng(96)
    lens, pos0 = [37, 1, 64, 100], [0, 50, 31, 200]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    B, T = len(lens), int(cu[-1])
    max_seq = 320
    w = synth.attn_weights(rng)
    tok = synth.attn_tokens(rng, T)
    kc = synth.normal_bf16(rng, (B, max_seq, nkv, d))
    vc = synth.normal_bf16(rng, (B, max_seq, nkv, d))
    layer = hip.attn_layer(dims, {k: _td(torch, v) for k, v in w.items()})
    t = {k: _td(torch, v) for k, v in tok.items()}

    def caches():
        dk = torch.empty((B, nkv, max_seq, d), dtype=torch.int16, device="cuda")
        dv = torch.empty((B, nkv, max_seq // 32, d, 32), dtype=torch.int16, device="cuda")
        for s in range(B):
            hip.attn_cache_pack(_td(torch, kc[s]), _td(torch, vc[s]), max_seq, nkv, d, dk[s],
                                dv[s], max_seq)
        return dk, dv

    dk1, dv1 = caches()
    y1 = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    hip.attn_prefill(layer, cu, pos0, t["qg"], t["k"], t["v"], dk1, dv1, max_seq, y1)
    dk2, dv2 = caches()
    y2 = torch.empty((T, nh * d), dtype=torch.int16, device="cuda")
    for s in range(B):
        a, b = int(cu[s]), int(cu[s + 1])
        hip.attn_prefill(layer, [0, b - a], [pos0[s]], t["qg"][a:b], t["k"][a:b], t["v"][a:b],
                         dk2[s:s + 1], dv2[s:s + 1], max_seq, y2[a:b])
    torch.cuda.synchronize()
    assert torch.equal(dk1, dk2) and torch.equal(dv1, dv2), "caches"
    assert torch.equal(y1, y2), "outputs"
