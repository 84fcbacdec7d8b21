"""Shared helpers for the attention parity tests: the per-element term
scale (esc) of the gated-GQA outputs, with an allowance for the rounding
decisions that a reordered score or probability sum may legitimately take
the other way.

The reference forms, per (query row, head) and key j (c/attn.h:337-368):
    s_j = q . k_j (fp32, ascending), A_j = rnd(rnd(s_j) * scale),
    P_j = rnd(e^{A_j - m} / sum e),  o_d = rnd(sum_j P_j V_jd).
Summed in another order (MFMA), s_j moves by at most the fp32 summation
bound gamma_n * sum_i |q_i k_ji| (n = d products, gamma_n = n * 2^-24). When
the exact s_j lies within twice that bound of a bf16 rounding midpoint,
either code is a correct rounding of a correctly ordered sum, and the two
differ by one bf16 ulp of s_j: P_j then moves by the factor e^{ulp * scale}.
Likewise P_j's own bf16 rounding flips when e/s lies within a few fp32
ulps of a midpoint (2^-8 of P_j). Each such j adds
|dP_j| * |V_jd| to what output d may deviate (and a flipped score,
renormalising the others, dP_j * esc_d); the allowance is passed to
numerics.assert_bf16_esc folded into esc (divided by its relative bar), so
the test bound per element is
    rel * (|r| + esc) + sum over flippable j of |dP_j| (|V_jd| + esc_d).
Everything else -- a wrong key, a dropped term, a mask off by one -- moves
an output by a whole P_j |V_jd| of a key that is not near a boundary, which
the bound does not cover.
"""
import numpy as np

from numerics import BF16_REL
from synth import bf16_f32

_U = 2.0 ** -24          # fp32 unit roundoff
_P_REL = 4e-6            # probability flip window (exp2 fold + divide)


def _midpoint_dist(x):
    """Distance of |x| from the nearest bf16 rounding midpoint, and the
    bf16 ulp at |x| (float64 arrays)."""
    ax = np.abs(x)
    e = np.floor(np.log2(np.maximum(ax, 1e-300)))
    ulp = np.exp2(e - 7)
    frac = ax / ulp - np.floor(ax / ulp)
    return np.abs(frac - 0.5) * ulp, ulp


def attn_esc_rows(qf_rows, K, V, qpos, nh, nkv, d, chunk=128, flips=True, rel=BF16_REL):
    """esc for some query rows of one sequence: qf_rows [n, nh*d] roped q
    codes, K, V [>= max(qpos)+1, nkv, d] cache codes after the append,
    qpos [n] the rows' positions (row i attends 0..qpos[i]). With flips,
    the rounding-flip allowance (module docstring) is folded in."""
    n = len(qpos)
    esc = np.zeros((n, nh, d))
    grp = nh // nkv
    scale = 1.0 / np.sqrt(d)
    for c0 in range(0, n, chunk):
        c1 = min(n, c0 + chunk)
        pos = np.asarray(qpos[c0:c1])
        npos = int(pos.max()) + 1
        q = bf16_f32(qf_rows[c0:c1]).astype(np.float64).reshape(c1 - c0, nh, d)
        masked = np.arange(npos)[None, None, :] > pos[:, None, None]
        for hk in range(nkv):
            Kf = bf16_f32(K[:npos, hk]).astype(np.float64)
            Vf = np.abs(bf16_f32(V[:npos, hk]).astype(np.float64))
            qh = q[:, hk * grp:(hk + 1) * grp]
            s = qh @ Kf.T                       # (BLAS; same values as the einsum)
            A = np.where(masked, -np.inf, s * scale)
            P = np.exp(A - A.max(2, keepdims=True))
            P /= P.sum(2, keepdims=True)
            e = P @ Vf
            if flips:
                tabs = np.abs(qh) @ np.abs(Kf).T
                dist, ulp = _midpoint_dist(s)
                sflip = dist <= 2.0 * d * _U * tabs
                dS = np.where(sflip & ~masked, P * np.expm1(ulp * scale), 0.0)
                pd, pulp = _midpoint_dist(P)
                pflip = (pd <= _P_REL * P) & ~masked
                dP = dS + np.where(pflip, pulp, 0.0)
                # a flipped score also renormalises every other P_k by
                # (1 - dS_j): up to dS_j * sum_k P_k |V_kd| = dS_j * esc
                allow = dP @ Vf + dS.sum(2, keepdims=True) * e
                e = e + allow * (1.02 / rel)
            esc[c0:c1, hk * grp:(hk + 1) * grp] = e
    return esc.reshape(n, nh * d)


def attn_esc(qf, kc, vc, cu, pos0, nh, nkv, d, flips=True):
    """esc per output element for a packed batch: qf [T, nh*d] roped q
    codes; kc, vc [B, max_seq, nkv, d] cache codes after the append. Token
    t of sequence s attends positions 0..pos0[s] + (t - cu[s])."""
    T = int(cu[-1])
    out = np.zeros((T, nh * d))
    for s in range(len(cu) - 1):
        t0, t1 = int(cu[s]), int(cu[s + 1])
        if t1 > t0:
            out[t0:t1] = attn_esc_rows(qf[t0:t1], kc[s], vc[s], pos0[s] + np.arange(t1 - t0),
                                       nh, nkv, d, flips=flips)
    return out
