"""Shared helpers for the attention parity tests."""
import numpy as np

from synth import bf16_f32


def attn_esc(qf, kc, vc, cu, pos0, nh, nkv, d, chunk=256):
    """esc = sum_j P_j |V_jd| per output element (the magnitude of the
    terms each output sums), P from the roped q and the cache in float64.
    qf [T, nh*d] roped q codes; kc, vc [B, max_seq, nkv, d] cache codes
    after the append. Token t of sequence s attends positions
    0..pos0[s] + (t - cu[s])."""
    T = int(cu[-1])
    esc = np.zeros((T, nh, d))
    grp = nh // nkv
    for s in range(len(cu) - 1):
        t0, t1 = int(cu[s]), int(cu[s + 1])
        for c0 in range(t0, t1, chunk):
            c1 = min(t1, c0 + chunk)
            pos = pos0[s] + np.arange(c0, c1) - t0            # query positions
            npos = int(pos[-1]) + 1
            q = bf16_f32(qf[c0:c1]).astype(np.float64).reshape(c1 - c0, nh, d)
            for hk in range(nkv):
                K = bf16_f32(kc[s, :npos, hk]).astype(np.float64)
                V = np.abs(bf16_f32(vc[s, :npos, hk]).astype(np.float64))
                A = np.einsum("thd,kd->thk", q[:, hk * grp:(hk + 1) * grp], K) / np.sqrt(d)
                A = np.where(np.arange(npos)[None, None, :] > pos[:, None, None], -np.inf, A)
                P = np.exp(A - A.max(2, keepdims=True))
                P /= P.sum(2, keepdims=True)
                esc[c0:c1, hk * grp:(hk + 1) * grp] = P @ V
    return esc.reshape(T, nh * d)
