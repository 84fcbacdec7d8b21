"""A synthetic hybrid model for the golden-stream harness.

The reference gates every engine change on a greedy token stream
(tests/m11/README.md: 24 greedy tokens after a short prompt, reproduced
bitwise). Its weights are absent here, so this harness builds a small model
of the same shape around the attention hot path: random weights, hidden
1024, four layers in the model's 3:1 ratio (three Gated DeltaNet layers,
then one gated-GQA layer; c/layer.h:236-331), each with the model's mixer
dims (GDN hk=16, hv=32, dk=dv=128; GQA nh=16, nkv=2, d=256, rot=64), a
(1+w) input RMSNorm, a residual, and a small dense SwiGLU MLP standing in
for the MoE block (out of the hot path).

Everything outside the mixers (embedding, norms, projections, MLP, lm head)
is the same numpy code on both paths, in float64; only the mixers' inputs
are rounded to bf16 codes (the C ABI's types), so two streams can differ
only through the mixers. (Rounding the residual stream to bf16 as well
would turn every ulp a mixer moves into fresh rounding flips downstream:
measured, it raises the logit noise of a one-ulp mixer difference about
tenfold, to the size of typical top-2 margins of a random model.) The mixers come from a backend:
  * OracleMixers -- the CPU restatement (or the reference's own compiled
    anchors through oracle.Reference), sequential per token;
  * HipMixers    -- the HIP library's tier-2 entry points (chunked GDN
    prefill, flash-attention prefill, fused GDN decode, split-K GQA decode,
    out-of-place GDN verify for speculative decoding).
This module is test infrastructure: the model around the mixers is not part
of the product.
"""
import numpy as np

import synth

H = 1024                   # hidden
V = 4096                   # vocab
FF = 512                   # MLP width
GD = synth.GDN_DIMS        # hk, hv, dk, dv
AD = synth.ATTN_DIMS       # nh, nkv, d, rot, theta
KINDS = ("gdn", "gdn", "gdn", "attn")
EPS = 1e-6


def rnd(x):
    """float64 -> bf16-valued float64 (RNE through fp32)."""
    return synth.bf16_f32(synth.bf16_bits(np.asarray(x, np.float32))).astype(np.float64)


def codes(x):
    return synth.bf16_bits(np.asarray(x, np.float32))


def _w(rng, shape, std):
    return rnd(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


class Model:
    """Weights of the synthetic model (seeded, identical on every machine)."""

    def __init__(self, seed=20260830):
        rng = np.random.default_rng(seed)
        hk, hv, dk, dv = GD
        nh, nkv, d = AD[0], AD[1], AD[2]
        self.cd = 2 * hk * dk + hv * dv
        self.embed = _w(rng, (V, H), 1.0)
        self.layers = []
        for kind in KINDS:
            L = dict(kind=kind, norm=_w(rng, (H,), 0.1), norm2=_w(rng, (H,), 0.1))
            if kind == "gdn":
                L["w_qkv"] = _w(rng, (H, self.cd), H ** -0.5)
                L["w_z"] = _w(rng, (H, hv * dv), H ** -0.5)
                L["w_ab"] = _w(rng, (H, 2 * hv), H ** -0.5)
                L["w_out"] = _w(rng, (hv * dv, H), (hv * dv) ** -0.5)
                L["mix"] = synth.gdn_weights(rng)
            else:
                L["w_qg"] = _w(rng, (H, nh * 2 * d), H ** -0.5)
                L["w_k"] = _w(rng, (H, nkv * d), H ** -0.5)
                L["w_v"] = _w(rng, (H, nkv * d), H ** -0.5)
                L["w_out"] = _w(rng, (nh * d, H), (nh * d) ** -0.5)
                L["mix"] = synth.attn_weights(rng)
            L["w_gate"] = _w(rng, (H, FF), H ** -0.5)
            L["w_up"] = _w(rng, (H, FF), H ** -0.5)
            L["w_down"] = _w(rng, (FF, H), FF ** -0.5)
            self.layers.append(L)
        self.norm_f = _w(rng, (H,), 0.1)
        self.lm_head = _w(rng, (H, V), H ** -0.5)


def rmsnorm(x, w):
    """(1+w) RMSNorm (the c/attn.h:175-186 form, row-wise), in float64."""
    rs = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + EPS)
    return x * rs * (1.0 + w)


def silu(x):
    return x / (1.0 + np.exp(-x))


def forward(model, mixers, cu, pos0, ids):
    """One engine step for a ragged batch: sequence s brings the tokens
    ids[cu[s]:cu[s+1]] at positions pos0[s]... Returns fp64 logits [T, V].
    The mixers advance their per-sequence state (conv, S, KV cache)."""
    hk, hv, dk, dv = GD
    nh, nkv, d = AD[0], AD[1], AD[2]
    h = model.embed[np.asarray(ids)]
    for li, L in enumerate(model.layers):
        x = rmsnorm(h, L["norm"])
        if L["kind"] == "gdn":
            qkv = codes(x @ L["w_qkv"])
            z = codes(x @ L["w_z"])
            ab = codes(x @ L["w_ab"])
            a = np.ascontiguousarray(ab[:, :hv])
            b = np.ascontiguousarray(ab[:, hv:])
            y = mixers.gdn(li, cu, qkv, z, a, b)
        else:
            qg = codes(x @ L["w_qg"])
            k = codes(x @ L["w_k"])
            v = codes(x @ L["w_v"])
            y = mixers.attn(li, cu, pos0, qg, k, v)
        h = h + synth.bf16_f32(y).astype(np.float64) @ L["w_out"]
        x2 = rmsnorm(h, L["norm2"])
        h = h + (silu(x2 @ L["w_gate"]) * (x2 @ L["w_up"])) @ L["w_down"]
    return rmsnorm(h, model.norm_f) @ model.lm_head


def greedy(logits):
    return np.argmax(logits, axis=-1)


def margin(logits):
    """top-1 minus top-2 logit per row."""
    p = np.sort(logits, axis=-1)
    return p[..., -1] - p[..., -2]


class OracleMixers:
    """Mixers on the CPU anchors: `orc` is oracle.Oracle() or
    oracle.Reference(); per-sequence states in the reference layouts."""

    def __init__(self, model, orc, B, max_seq):
        self.m, self.orc, self.max_seq = model, orc, max_seq
        hk, hv, dk, dv = GD
        nkv, d = AD[1], AD[2]
        self.conv = {}
        self.S = {}
        self.kc = {}
        self.vc = {}
        for li, L in enumerate(model.layers):
            if L["kind"] == "gdn":
                self.conv[li] = np.zeros((B, model.cd * 3), np.uint16)
                self.S[li] = np.zeros((B, hv, dk, dv), np.float32)
            else:
                self.kc[li] = np.zeros((B, max_seq, nkv, d), np.uint16)
                self.vc[li] = np.zeros((B, max_seq, nkv, d), np.uint16)

    def gdn(self, li, cu, qkv, z, a, b):
        return self.orc.gdn_mixer(GD, self.m.layers[li]["mix"], np.asarray(cu, np.int32),
                                  qkv, z, a, b, self.conv[li], self.S[li])

    def attn(self, li, cu, pos0, qg, k, v):
        nkv, d = AD[1], AD[2]
        return self.orc.attn_mixer(AD, self.m.layers[li]["mix"], np.asarray(cu, np.int32),
                                   np.asarray(pos0, np.int32), qg, k, v, self.kc[li],
                                   self.vc[li], self.max_seq * nkv * d)


class HipMixers:
    """Mixers on the HIP library (device-resident state and caches).

    A step in which some sequence brings more than 4 tokens (a prompt) runs
    the chunked GDN prefill and the flash-attention prefill; decode steps
    (1..4 tokens per sequence) run the fused GDN decode and the split-K GQA
    decode. With spec=True every GDN
    layer keeps two state sets and verifies out of place
    (apus_hip_gdn_decode_into), so a rejected draft is rolled back by
    re-feeding the accepted prefix from the untouched set."""

    def __init__(self, model, hip, B, max_seq, spec=False):
        import torch
        self.torch, self.hip, self.m, self.B = torch, hip, model, B
        self.max_seq = max_seq
        self.spec = spec
        dev = torch.device("cuda")
        self.dev = dev
        hk, hv, dk, dv = GD
        nkv, d = AD[1], AD[2]

        def t(a):
            a = np.ascontiguousarray(a)
            return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)
        self.t = t
        self.layer = {}
        self.conv, self.S = {}, {}
        self.kc, self.vc = {}, {}
        for li, L in enumerate(model.layers):
            if L["kind"] == "gdn":
                self.layer[li] = hip.gdn_layer(GD, {n: t(v) for n, v in L["mix"].items()})
                sets = 2 if spec else 1
                self.conv[li] = [torch.zeros((B, model.cd * 3), dtype=torch.int16, device=dev)
                                 for _ in range(sets)]
                self.S[li] = [torch.zeros((B, hv, dk, dv), dtype=torch.float32, device=dev)
                              for _ in range(sets)]
            else:
                self.layer[li] = hip.attn_layer(AD, {n: t(v) for n, v in L["mix"].items()})
                self.kc[li] = torch.zeros((B, nkv, max_seq, d), dtype=torch.int16, device=dev)
                self.vc[li] = torch.zeros((B, nkv, max_seq // 32, d, 32), dtype=torch.int16,
                                          device=dev)
        self.live = 0              # index of the live GDN state set (spec mode)
        self.verify = False        # spec mode: GDN steps verify out of place

    def _y(self, T, n):
        return self.torch.empty((T, n), dtype=self.torch.int16, device=self.dev)

    def gdn(self, li, cu, qkv, z, a, b):
        hv, dv = GD[1], GD[3]
        cu = np.asarray(cu, np.int32)
        T = int(cu[-1])
        tq, tz, ta, tb = (self.t(x) for x in (qkv, z, a, b))
        y = self._y(T, hv * dv)
        multi = int(np.max(np.diff(cu))) > 4
        if self.verify:
            src, dst = self.live, 1 - self.live
            self.hip.gdn_decode_into(self.layer[li], cu, tq, tz, ta, tb,
                                     self.conv[li][src], self.S[li][src],
                                     self.conv[li][dst], self.S[li][dst], y)
        elif multi:
            self.hip.gdn_prefill(self.layer[li], cu, tq, tz, ta, tb, self.conv[li][self.live],
                                 self.S[li][self.live], y)
        else:
            self.hip.gdn_decode(self.layer[li], cu, tq, tz, ta, tb, self.conv[li][self.live],
                                self.S[li][self.live], y)
        self.torch.cuda.synchronize()
        return y.cpu().numpy().view(np.uint16)

    def gdn_refeed(self, li, cu, qkv, z, a, b):
        """Spec mode: re-feed accepted prefixes from the live (snapshot) set
        into the other set; sequences with no tokens keep their verify
        state there."""
        hv, dv = GD[1], GD[3]
        cu = np.asarray(cu, np.int32)
        src, dst = self.live, 1 - self.live
        if int(cu[-1]) == 0:
            return
        y = self._y(int(cu[-1]), hv * dv)
        self.hip.gdn_decode_into(self.layer[li], cu, *(self.t(x) for x in (qkv, z, a, b)),
                                 self.conv[li][src], self.S[li][src],
                                 self.conv[li][dst], self.S[li][dst], y)

    def commit(self):
        """Spec mode: the verified set becomes the live one."""
        self.live = 1 - self.live

    def attn(self, li, cu, pos0, qg, k, v):
        nh, d = AD[0], AD[2]
        cu = np.asarray(cu, np.int32)
        T = int(cu[-1])
        y = self._y(T, nh * d)
        args = (self.layer[li], cu, np.asarray(pos0, np.int32), self.t(qg), self.t(k),
                self.t(v), self.kc[li], self.vc[li], self.max_seq, y)
        if int(np.max(np.diff(cu))) > 4:
            self.hip.attn_prefill(*args)
        else:
            self.hip.attn_decode(*args)
        self.torch.cuda.synchronize()
        return y.cpu().numpy().view(np.uint16)


def run_greedy(model, mixers, prompts, n_new, forced=None):
    """Prefill the prompts as one ragged batch, then n_new - 1 decode steps
    of one token per sequence. Each step feeds the argmax of the previous
    step, or forced[:, i] when given (teacher forcing, so that two backends
    are compared step by step on the same inputs). Returns (ids, logits):
    the argmax ids [B, n_new] and the logits behind them [B, n_new, V]."""
    B = len(prompts)
    lens = np.array([len(p) for p in prompts], np.int32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    logits = forward(model, mixers, cu, np.zeros(B, np.int32), np.concatenate(prompts))
    last = logits[cu[1:] - 1]
    ids = np.zeros((B, n_new), np.int64)
    lg = np.zeros((B, n_new, V))
    pos = lens.copy()
    one = np.arange(B + 1, dtype=np.int32)
    for i in range(n_new):
        ids[:, i] = greedy(last)
        lg[:, i] = last
        if i + 1 == n_new:
            break
        feed = ids[:, i] if forced is None else np.asarray(forced)[:, i]
        last = forward(model, mixers, one, pos, feed)
        pos += 1
    return ids, lg


def run_speculative(model, hip_mixers, prompts, n_new, drafts):
    """Greedy decoding with MTP-style verification on the HIP mixers: each
    step feeds the last accepted token plus up to 3 draft tokens per
    sequence (drafts(s, i) gives the draft for sequence s at output index i),
    accepts the longest prefix the model agrees with, and rolls the GDN
    state back to it (re-feed from the snapshot set); full-attention layers
    roll back by position alone. Returns the generated ids [B, n_new], which
    must equal plain greedy decoding."""
    B = len(prompts)
    lens = np.array([len(p) for p in prompts], np.int32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    m = hip_mixers
    logits = forward(model, m, cu, np.zeros(B, np.int32), np.concatenate(prompts))
    first = greedy(logits[cu[1:] - 1])
    out = [[int(first[s])] for s in range(B)]
    pos = lens.copy()
    while min(len(o) for o in out) < n_new:
        # step input per sequence: the last accepted token + drafts
        feeds = []
        for s in range(B):
            n = len(out[s])
            k = min(3, max(0, n_new - n))
            feeds.append([out[s][-1]] + [int(drafts(s, n + j)) for j in range(k)])
        k_s = np.array([len(f) for f in feeds], np.int32)
        vcu = np.concatenate([[0], np.cumsum(k_s)]).astype(np.int32)
        ids = np.concatenate([np.array(f, np.int64) for f in feeds])
        # the verify pass writes the other GDN set; remember the mixer
        # inputs for a re-feed
        captured = {}
        orig_gdn = m.gdn

        def cap_gdn(li, cu_, qkv, z, a, b):
            captured[li] = (qkv, z, a, b)
            return orig_gdn(li, cu_, qkv, z, a, b)
        m.gdn = cap_gdn
        m.verify = True
        logits = forward(model, m, vcu, pos, ids)
        m.verify = False
        m.gdn = orig_gdn
        pred = greedy(logits)
        acc = np.zeros(B, np.int32)          # fed tokens kept per sequence
        for s in range(B):
            p = pred[vcu[s]:vcu[s + 1]]
            f = feeds[s]
            j = 0
            while j + 1 < len(f) and f[j + 1] == p[j]:
                j += 1
            acc[s] = j + 1                   # the last token and j drafts
            for t in range(j + 1):
                if len(out[s]) < n_new:
                    out[s].append(int(p[t]))
        # roll back sequences that rejected a draft: re-feed their accepted
        # prefix from the snapshot into the verify set
        rcu = np.zeros(B + 1, np.int32)
        rows = []
        for s in range(B):
            n = int(acc[s]) if acc[s] < k_s[s] else 0
            rcu[s + 1] = rcu[s] + n
            rows += list(range(vcu[s], vcu[s] + n))
        for li, (qkv, z, a, b) in captured.items():
            m.gdn_refeed(li, rcu, qkv[rows], z[rows], a[rows], b[rows])
        m.commit()
        pos += acc
    return np.array([o[:n_new] for o in out], np.int64)
