"""GPU tests of the serving-side state managers: the paged KV cache
(apus_hip_kv_pool_*, apus_hip_attn_{decode,prefill}_paged) and the GDN state
pool (apus_hip_gdn_pool_*, apus_hip_gdn_{decode,prefill}_slots).

The paged and slotted entry points run the same kernels as the flat ones
with a different address map, so on the same inputs their outputs and
states are held BIT-EXACT to the flat path (same split plan, same summation
order), which the flat tests hold to the oracle; one case per entry point
is also checked against the oracle directly. Blocks are handed out in a
shuffled order so a sequence's blocks are scattered over the pool, and
sequences grow across block boundaries between steps.
"""
import numpy as np
import pytest

import synth
from attn_util import attn_esc_rows
from numerics import assert_bf16_close, assert_bf16_esc, assert_state_close

pytestmark = pytest.mark.gpu

NH, NKV, D, ROT, THETA = synth.ATTN_DIMS
GD = synth.GDN_DIMS


def _td(torch, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to("cuda")


def _h(t):
    return t.cpu().numpy().view(np.uint16)


def test_paged_decode_matches_flat(hip, orc):
    """Ragged decode/verify over 40 sequences (contexts 1..3000, 1..4 new
    tokens) on a paged cache whose blocks are scattered, three steps with
    growth across block boundaries: bit-exact to the flat cache, and the
    first step against the oracle."""
    import torch
    rng = np.random.default_rng(31)
    B = 40
    ctx = rng.integers(1, 3000, B).astype(np.int32)
    steps = [rng.integers(1, 5, B).astype(np.int32) for _ in range(3)]
    final = ctx + sum(steps)
    max_seq = int(-(-int(final.max()) // 32) * 32)
    nblocks = int(np.sum(-(-final // 32))) + 64
    pool = hip.KvPool(1, NKV, D, nblocks, B + 8, max_seq // 32)
    # scatter the free list: rows reserve one block at a time round-robin
    rows = [pool.open() for _ in range(B)]
    order = rng.permutation(B)
    have = np.zeros(B, np.int64)
    need = -(-ctx // 32)
    while (have < need).any():
        for s in order:
            if have[s] < need[s]:
                have[s] += 1
                pool.reserve(rows[s], int(have[s]) * 32 if have[s] < need[s] else int(ctx[s]))
    kv = pool.cache(0)
    w = synth.attn_weights(rng)
    layer = hip.attn_layer(synth.ATTN_DIMS, {n: _td(torch, a) for n, a in w.items()})
    dk = torch.zeros((B, NKV, max_seq, D), dtype=torch.int16, device="cuda")
    dv = torch.zeros((B, NKV, max_seq // 32, D, 32), dtype=torch.int16, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(31)
    hk_list, hv_list = [], []
    for s in range(B):
        kr = (torch.randn((int(ctx[s]), NKV, D), generator=g, device="cuda")).to(torch.bfloat16).view(torch.int16)
        vr = (torch.randn((int(ctx[s]), NKV, D), generator=g, device="cuda")).to(torch.bfloat16).view(torch.int16)
        hip.attn_cache_pack(kr, vr, int(ctx[s]), NKV, D, dk[s], dv[s], max_seq)
        hip.attn_cache_pack_paged(kr, vr, int(ctx[s]), NKV, D, kv, rows[s])
        hk_list.append(_h(kr))
        hv_list.append(_h(vr))
    pos = ctx.copy()
    for i, k in enumerate(steps):
        cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
        T = int(cu[-1])
        for s in range(B):
            pool.reserve(rows[s], int(pos[s] + k[s]))
        tok = synth.attn_tokens(rng, T)
        t = {n: _td(torch, a) for n, a in tok.items()}
        y1 = torch.empty((T, NH * D), dtype=torch.int16, device="cuda")
        y2 = torch.empty_like(y1)
        hip.attn_decode(layer, cu, pos, t["qg"], t["k"], t["v"], dk, dv, max_seq, y1)
        hip.attn_decode_paged(layer, rows, cu, pos, t["qg"], t["k"], t["v"], kv, y2)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), f"step {i}: paged decode differs from flat"
        if i == 0:
            off = np.concatenate([[0], np.cumsum((ctx + k).astype(np.int64) * NKV * D)])
            hkk = np.concatenate([np.concatenate([hk_list[s].reshape(-1),
                                                  np.zeros(int(k[s]) * NKV * D, np.uint16)])
                                  for s in range(B)])
            hvv = np.concatenate([np.concatenate([hv_list[s].reshape(-1),
                                                  np.zeros(int(k[s]) * NKV * D, np.uint16)])
                                  for s in range(B)])
            y_o, qf, _, _ = orc.attn_mixer_off(synth.ATTN_DIMS, w, cu, pos, tok["qg"], tok["k"],
                                               tok["v"], hkk, hvv, off[:-1], nthreads=16,
                                               capture=True)
            esc = np.concatenate([
                attn_esc_rows(qf[cu[s]:cu[s + 1]], hkk[off[s]:off[s + 1]].reshape(-1, NKV, D),
                              hvv[off[s]:off[s + 1]].reshape(-1, NKV, D),
                              pos[s] + np.arange(k[s]), NH, NKV, D) for s in range(B)])
            print("[paged decode] vs oracle", assert_bf16_esc(_h(y2), y_o, esc, ulps=2,
                                                              what="paged decode y"), flush=True)
        pos = pos + k
    # the whole caches agree
    for s in range(B):
        n = int(pos[s])
        a = [torch.empty((n, NKV, D), dtype=torch.int16, device="cuda") for _ in range(4)]
        hip.attn_cache_unpack(dk[s], dv[s], n, NKV, D, max_seq, a[0], a[1])
        hip.attn_cache_unpack_paged(kv, rows[s], n, NKV, D, a[2], a[3])
        torch.cuda.synchronize()
        assert torch.equal(a[0], a[2]) and torch.equal(a[1], a[3]), f"cache of sequence {s}"
    used = nblocks - pool.free_blocks()
    assert used == int(np.sum(-(-pos // 32))), "blocks held = blocks the positions need"
    for r in rows:
        pool.close(r)
    assert pool.free_blocks() == nblocks
    pool.destroy()


def test_paged_prefill_matches_flat(hip, orc):
    """Ragged prefill (new sequences and continuations after a cached prefix)
    on scattered paged blocks: bit-exact to the flat cache; against the
    oracle."""
    import torch
    rng = np.random.default_rng(32)
    lens = np.array([37, 200, 1, 96, 513, 64], np.int32)
    pre = np.array([0, 0, 50, 31, 0, 700], np.int32)
    B = len(lens)
    final = pre + lens
    max_seq = int(-(-int(final.max()) // 32) * 32)
    pool = hip.KvPool(1, NKV, D, 400, 16, max_seq // 32)
    rows = [pool.open() for _ in range(B)]
    # interleave the reservations so blocks alternate between rows
    for b in range(1, max_seq // 32 + 1):
        for s in rng.permutation(B):
            if (b - 1) * 32 < final[s]:
                pool.reserve(rows[s], min(b * 32, int(final[s])))
    kv = pool.cache(0)
    w = synth.attn_weights(rng)
    layer = hip.attn_layer(synth.ATTN_DIMS, {n: _td(torch, a) for n, a in w.items()})
    dk = torch.zeros((B, NKV, max_seq, D), dtype=torch.int16, device="cuda")
    dv = torch.zeros((B, NKV, max_seq // 32, D, 32), dtype=torch.int16, device="cuda")
    kc = synth.normal_bf16(rng, (B, max_seq, NKV, D))
    vc = synth.normal_bf16(rng, (B, max_seq, NKV, D))
    for s in range(B):
        if pre[s]:
            a, b = _td(torch, kc[s, :pre[s]]), _td(torch, vc[s, :pre[s]])
            hip.attn_cache_pack(a, b, int(pre[s]), NKV, D, dk[s], dv[s], max_seq)
            hip.attn_cache_pack_paged(a, b, int(pre[s]), NKV, D, kv, rows[s])
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    tok = synth.attn_tokens(rng, T)
    t = {n: _td(torch, a) for n, a in tok.items()}
    y1 = torch.empty((T, NH * D), dtype=torch.int16, device="cuda")
    y2 = torch.empty_like(y1)
    hip.attn_prefill(layer, cu, pre, t["qg"], t["k"], t["v"], dk, dv, max_seq, y1)
    hip.attn_prefill_paged(layer, rows, cu, pre, t["qg"], t["k"], t["v"], kv, y2)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "paged prefill differs from flat"
    k_o, v_o = kc.copy(), vc.copy()
    y_o, qf, _ = orc.attn_mixer(synth.ATTN_DIMS, w, cu, pre, tok["qg"], tok["k"], tok["v"], k_o,
                                v_o, max_seq * NKV * D, capture=True)
    esc = np.concatenate([attn_esc_rows(qf[cu[s]:cu[s + 1]], k_o[s], v_o[s],
                                        pre[s] + np.arange(lens[s]), NH, NKV, D)
                          for s in range(B)])
    print("[paged prefill]", assert_bf16_esc(_h(y2), y_o, esc, ulps=2, what="paged prefill y"))
    for s in range(B):
        n = int(final[s])
        rk = torch.empty((n, NKV, D), dtype=torch.int16, device="cuda")
        rv = torch.empty_like(rk)
        hip.attn_cache_unpack_paged(kv, rows[s], n, NKV, D, rk, rv)
        torch.cuda.synchronize()
        assert np.array_equal(_h(rk), k_o[s, :n]) and np.array_equal(_h(rv), v_o[s, :n])
    pool.destroy()


def test_kv_pool_bookkeeping(hip):
    """Rows and blocks are recycled; exhaustion and over-long reservations
    are refused with an error (no state change)."""
    pool = hip.KvPool(2, NKV, D, 10, 3, 4)
    a, b = pool.open(), pool.open()
    pool.reserve(a, 100)                     # 4 blocks
    pool.reserve(b, 33)                      # 2 blocks
    assert pool.free_blocks() == 4
    with pytest.raises(hip.ApusHipError):
        pool.reserve(b, 129)                 # beyond max_blocks (4 per row)
    c = pool.open()
    with pytest.raises(hip.ApusHipError):
        pool.reserve(c, 160)                 # > free blocks and > max_blocks
    pool.reserve(c, 128)                     # exactly the 4 free blocks
    assert pool.free_blocks() == 0
    with pytest.raises(hip.ApusHipError):
        pool.open()                          # no free row
    pool.close(a)
    assert pool.free_blocks() == 4
    d = pool.open()
    pool.reserve(d, 1)
    assert pool.free_blocks() == 3
    k0, k1 = pool.cache(0), pool.cache(1)
    assert k0.k != k1.k and k0.block_table == k1.block_table
    pool.destroy()


def test_paged_rows_checked(hip):
    """A paged call naming a row outside the block table, a closed row, or
    positions past the blocks its row reserved is refused before any
    kernel runs (the stale table entries of a closed row would otherwise
    point into another sequence's blocks)."""
    import torch
    rng = np.random.default_rng(77)
    layer = hip.attn_layer(synth.ATTN_DIMS, {n: torch.from_numpy(v.view(np.int16)).cuda()
                                            for n, v in synth.attn_weights(rng).items()})
    tok = {n: torch.from_numpy(v.view(np.int16)).cuda() for n, v in synth.attn_tokens(rng, 1).items()}
    y = torch.empty((1, synth.ATTN_DIMS[0] * D), dtype=torch.int16, device="cuda")
    pool = hip.KvPool(1, NKV, D, 8, 3, 4)
    a, b = pool.open(), pool.open()
    pool.reserve(a, 64)                      # 2 blocks: positions 0..63
    pool.reserve(b, 40)
    kv = pool.cache(0)
    hip.attn_decode_paged(layer, [a], [0, 1], [63], tok["qg"], tok["k"], tok["v"], kv, y)
    torch.cuda.synchronize()
    for rows, pos0, why in (([3], [0], "row past the table"), ([-1], [0], "negative row"),
                            ([a], [64], "position past the reserved blocks"),
                            ([b], [64], "position past the reserved blocks")):
        with pytest.raises(hip.ApusHipError) as e:
            hip.attn_decode_paged(layer, rows, [0, 1], pos0, tok["qg"], tok["k"], tok["v"], kv, y)
        assert e.value.code == 3, why
    pool.close(b)
    with pytest.raises(hip.ApusHipError):
        hip.attn_decode_paged(layer, [b], [0, 1], [0], tok["qg"], tok["k"], tok["v"], kv, y)
    with pytest.raises(hip.ApusHipError):      # the prefill form checks the same
        hip.attn_prefill_paged(layer, [a], [0, 1], [64], tok["qg"], tok["k"], tok["v"], kv, y)
    pool.destroy()


def _gdn_inputs(rng, T):
    return synth.gdn_tokens(rng, T)


def test_gdn_slots_match_flat(hip, orc):
    """Prefill then two decode/verify steps of 5 sequences living at
    scattered slots of a 12-slot pool: bit-exact to the flat path on states
    packed in batch order; a new slot starts at zero state; the prefill is
    checked against the oracle."""
    import torch
    rng = np.random.default_rng(33)
    B = 5
    pool = hip.GdnPool(1, GD, 12)
    junk = [pool.open() for _ in range(4)]          # occupy some slots first
    slots = [pool.open() for _ in range(B)]
    for j in junk[1:3]:
        pool.close(j)
    conv_b, S_b = pool.state(0)
    hk, hv, dk, dvv = GD
    cd = 2 * hk * dk + hv * dvv
    w = synth.gdn_weights(rng)
    layer = hip.gdn_layer(GD, {n: _td(torch, a) for n, a in w.items()})
    # flat reference states, zero like a freshly opened slot
    fconv = torch.zeros((B, cd * 3), dtype=torch.int16, device="cuda")
    fS = torch.zeros((B, hv, dk, dvv), dtype=torch.float32, device="cuda")
    lens = np.array([70, 1, 130, 64, 5], np.int32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    tok = _gdn_inputs(rng, int(cu[-1]))
    t = {n: _td(torch, a) for n, a in tok.items()}
    y1 = torch.empty((int(cu[-1]), hv * dvv), dtype=torch.int16, device="cuda")
    y2 = torch.empty_like(y1)
    hip.gdn_prefill(layer, cu, t["qkv"], t["z"], t["a"], t["b"], fconv, fS, y1)
    hip.gdn_prefill_slots(layer, slots, cu, t["qkv"], t["z"], t["a"], t["b"], conv_b, S_b, y2)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "slotted prefill output differs"
    elem = hv * dk * dvv

    def slot_state(slot):
        """A slot's conv state and S, copied back through the C ABI."""
        import ctypes
        torch.cuda.synchronize()
        hc = np.empty(cd * 3, np.uint16)
        hS = np.empty(elem, np.float32)
        for dst, src in ((hc, conv_b + slot * cd * 3 * 2), (hS, S_b + slot * elem * 4)):
            hip._chk(hip.load().apus_hip_memcpy_d2h(dst.ctypes.data_as(ctypes.c_void_p),
                                                    ctypes.c_void_p(src),
                                                    ctypes.c_size_t(dst.nbytes)))
        return hc, hS

    for i, s in enumerate(slots):
        hc, hS = slot_state(s)
        assert np.array_equal(hc, _h(fconv[i])), f"conv state of slot {s}"
        assert np.array_equal(hS, fS[i].reshape(-1).cpu().numpy()), f"S of slot {s}"
    c_o = np.zeros((B, cd * 3), np.uint16)
    S_o = np.zeros((B, hv, dk, dvv), np.float32)
    y_o = orc.gdn_mixer(GD, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], c_o, S_o, nthreads=16)
    from numerics import assert_bf16_rows
    assert_bf16_rows(_h(y2), y_o, hv * dvv, what="slotted prefill y")

    # decode in place, then out of place into fresh slots (an MTP snapshot)
    for step in range(2):
        k = rng.integers(1, 5, B).astype(np.int32)
        cu2 = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
        tok = _gdn_inputs(rng, int(cu2[-1]))
        t = {n: _td(torch, a) for n, a in tok.items()}
        y1 = torch.empty((int(cu2[-1]), hv * dvv), dtype=torch.int16, device="cuda")
        y2 = torch.empty_like(y1)
        if step == 0:
            hip.gdn_decode(layer, cu2, t["qkv"], t["z"], t["a"], t["b"], fconv, fS, y1)
            hip.gdn_decode_slots(layer, slots, slots, cu2, t["qkv"], t["z"], t["a"], t["b"],
                                 conv_b, S_b, y2)
        else:
            outs = [pool.open() for _ in range(B)]
            fconv2, fS2 = torch.empty_like(fconv), torch.empty_like(fS)
            hip.gdn_decode_into(layer, cu2, t["qkv"], t["z"], t["a"], t["b"], fconv, fS, fconv2,
                                fS2, y1)
            hip.gdn_decode_slots(layer, slots, outs, cu2, t["qkv"], t["z"], t["a"], t["b"],
                                 conv_b, S_b, y2)
            fconv_keep, fS_keep = fconv, fS
            fconv, fS = fconv2, fS2
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), f"slotted decode step {step} differs"
    for i in range(B):
        hc, hS = slot_state(outs[i])
        assert np.array_equal(hc, _h(fconv[i])) and np.array_equal(hS, fS[i].reshape(-1).cpu().numpy())
        hc, hS = slot_state(slots[i])                # the snapshot is untouched
        assert np.array_equal(hc, _h(fconv_keep[i]))
        assert np.array_equal(hS, fS_keep[i].reshape(-1).cpu().numpy())
    # a reopened slot is zero again
    pool.close(outs[0])
    z = pool.open()
    hc, hS = slot_state(z)
    assert not hc.any() and not hS.any()
    pool.destroy()


def test_gdn_slot_maps_rejected(hip):
    """Slot maps that would let one sequence's writes reach another's state
    are refused before any launch."""
    import torch
    rng = np.random.default_rng(34)
    pool = hip.GdnPool(1, GD, 6)
    conv_b, S_b = pool.state(0)
    w = synth.gdn_weights(rng)
    layer = hip.gdn_layer(GD, {n: _td(torch, a) for n, a in w.items()})
    tok = _gdn_inputs(rng, 2)
    t = {n: _td(torch, a) for n, a in tok.items()}
    y = torch.empty((2, GD[1] * GD[3]), dtype=torch.int16, device="cuda")
    cu = [0, 1, 2]
    for si, so in (([0, 1], [2, 2]),      # two writers of one slot
                   ([0, 1], [1, 3])):     # sequence 0 writes sequence 1's input
        with pytest.raises(hip.ApusHipError):
            hip.gdn_decode_slots(layer, si, so, cu, t["qkv"], t["z"], t["a"], t["b"], conv_b,
                                 S_b, y)
    with pytest.raises(hip.ApusHipError):
        hip.gdn_prefill_slots(layer, [3, 3], cu, t["qkv"], t["z"], t["a"], t["b"], conv_b, S_b, y)
    pool.destroy()
