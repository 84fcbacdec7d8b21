"""Tolerance checks shared by the parity tests.

Tolerances (made precise here):
  * bf16 outputs: relative error ||c - r||_2 / ||r||_2 <= 2e-3 over the
    tensor, and no element further than `max_ulp` bf16 ulps from the
    oracle (1 for ops that keep the reference's summation order, where a
    difference can only come from a libm ulp or a summation-order ulp
    crossing a bf16 rounding boundary) unless its absolute difference is
    below 1e-3 of the tensor's rms (values that are tiny through
    cancellation, where an upstream fp32 ulp moves several bf16 ulps).
  * fp32 recurrent state: max |c - r| / max |r| <= 1e-4.
  * integer-like data (codes of exact copies, cache rows): bit-exact.
"""
import numpy as np

BF16_REL = 2e-3
STATE_REL = 1e-4


def _ordered(codes):
    """Map bf16 codes to integers whose difference is the ulp distance."""
    c = np.asarray(codes, dtype=np.uint16).astype(np.int32)
    return np.where(c & 0x8000, 0x8000 - c, c)


def ulp_diff(a, b):
    return np.abs(_ordered(a) - _ordered(b))


def f32_of(codes):
    return (np.asarray(codes, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_stats(c, r):
    c = np.asarray(c).ravel()
    r = np.asarray(r).ravel()
    cf = f32_of(c).astype(np.float64)
    rf = f32_of(r).astype(np.float64)
    nr = np.linalg.norm(rf)
    rel = np.linalg.norm(cf - rf) / nr if nr > 0 else np.linalg.norm(cf)
    ud = ulp_diff(c, r)
    rms = np.sqrt(np.mean(rf * rf)) if rf.size else 0.0
    far = np.abs(cf - rf) > 1e-3 * rms
    return dict(rel=float(rel), max_ulp=int(ud[far].max()) if far.any() else int(min(1, ud.max(initial=0))),
                exact=float(np.mean(ud == 0)) if ud.size else 1.0, n=int(ud.size),
                raw_max_ulp=int(ud.max(initial=0)))


def assert_bf16_close(c, r, max_ulp=1, rel=BF16_REL, what=""):
    st = bf16_stats(c, r)
    assert st["rel"] <= rel and st["max_ulp"] <= max_ulp, f"{what}: {st}"
    return st


def state_rel(c, r):
    c = np.asarray(c, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    den = np.max(np.abs(r))
    return float(np.max(np.abs(c - r)) / den) if den > 0 else float(np.max(np.abs(c)))


def assert_state_close(c, r, rel=STATE_REL, what=""):
    e = state_rel(c, r)
    assert e <= rel, f"{what}: state rel err {e:.3g} > {rel}"
    return e


def f32_stats(c, r):
    c = np.asarray(c, np.float32).ravel()
    r = np.asarray(r, np.float32).ravel()
    same = np.mean(c.view(np.uint32) == r.view(np.uint32)) if c.size else 1.0
    return dict(exact=float(same), rel=state_rel(c, r))


def assert_bf16_esc(c, r, esc, rel=BF16_REL, ulps=1, what=""):
    """Tolerance class for reordered reductions (the reference's own form,
    tests/m4a/test_gdn.c:84-95): every element within `ulps` bf16 ulps of
    the reference, or |c - r| <= rel*(|r| + esc) with esc the sum of |terms| of
    that output; and ||c - r||_2/||r||_2 <= rel over the tensor. Outputs
    that are small through cancellation (|r| << esc) are judged against the
    size of their terms, as the reference judges its own; the one-ulp
    allowance is the final bf16 rounding itself (a single ulp is already
    2^-8..2^-7 relative, so an fp32 value within rel*esc of the reference's
    can still round to the neighbouring code when one term dominates; a
    later rounding point, such as the output gate's rnd(o * g), can carry
    that one ulp of o into two ulps of its result)."""
    st = bf16_stats(c, r)
    cf = f32_of(np.asarray(c).ravel()).astype(np.float64)
    rf = f32_of(np.asarray(r).ravel()).astype(np.float64)
    e = np.asarray(esc, np.float64).ravel()
    ratio = np.abs(cf - rf) / (np.abs(rf) + e + 1e-30)
    ud = ulp_diff(np.asarray(c).ravel(), np.asarray(r).ravel())
    judged = ud > ulps
    st["esc_max"] = float(ratio[judged].max()) if judged.any() else 0.0
    st["esc_max_all"] = float(ratio.max()) if ratio.size else 0.0
    assert st["rel"] <= rel and st["esc_max"] <= rel, f"{what}: {st}"
    return st


def assert_bf16_rows(c, r, ncols, max_ulp=4, rel=BF16_REL, floor=BF16_REL, abs_floor=1e-5,
                     what=""):
    """Tolerance class for a reordered fp32 reduction feeding bf16 rounding
    points and a per-row normalisation (the chunked GDN output: o from the
    chunk form, rnd(o), then the gated RMSNorm's three roundings,
    c/gdn.h:639-661). An fp32 ulp of o that crosses a bf16 boundary moves
    rnd(o) by one ulp and each later rounding by at most one more, so an
    element may sit up to 4 ulps away; elements small through cancellation
    (|c - r| <= floor * rms of their row) are judged against the row's
    scale instead. Rows whose recurrence output lies below the norm's eps
    (a state decayed to ~0) are o * rs with rs up to 1/sqrt(1e-6): their
    values are amplified fp32 noise of a near-zero o, so differences under
    abs_floor * rms of the whole tensor are not counted either.
    Normwise ||c - r||_2 / ||r||_2 <= rel over the tensor."""
    st = bf16_stats(c, r)
    c2 = np.asarray(c).reshape(-1, ncols)
    r2 = np.asarray(r).reshape(-1, ncols)
    cf = f32_of(c2).astype(np.float64)
    rf = f32_of(r2).astype(np.float64)
    rms = np.sqrt(np.mean(rf * rf, axis=1, keepdims=True))
    grms = np.sqrt(np.mean(rf * rf)) if rf.size else 0.0
    far = np.abs(cf - rf) > np.maximum(floor * rms, abs_floor * grms)
    ud = ulp_diff(c2, r2)
    st["max_ulp"] = int(ud[far].max()) if far.any() else 0
    assert st["rel"] <= rel and st["max_ulp"] <= max_ulp, f"{what}: {st}"
    return st
