"""The oracle (and the HIP tier-1 ops) against golden vectors written by the
reference's own scalar anchors (tests/golden/make_golden.py, compiled from
c/gdn.h, c/attn.h, c/bf16.h and wired as c/layer.h).

These pin the oracle bit for bit without /root/reference at test time:
every op and both mixers (at reduced dims) must reproduce the reference's
output codes / fp32 bits exactly. The GPU half replays the single-op
vectors through the C ABI with the tier-1 tolerance (bitwise but for libm
ulps crossing a rounding boundary).
"""
import os

import numpy as np
import pytest

from numerics import assert_bf16_close, assert_state_close

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def gv():
    with np.load(GOLD) as f:
        return {k: f[k] for k in f.files}


def _ops_outputs(ops, v):
    """Run the single-op cases through `ops` (oracle or HIP binding)."""
    out = {}
    st = v["conv_state0"].copy()
    out["conv_out"] = ops.gdn_conv1d(v["conv_x"], v["conv_w"], st)
    out["conv_state1"] = st
    out["decay_g"] = ops.gdn_decay(v["gate_a"], v["gate_A_log"], v["gate_dt"])
    out["beta"] = ops.gdn_beta(v["gate_b"])
    out["l2_y"] = ops.gdn_l2norm(v["l2_x"], 3, 16, 16 ** -0.5)
    T, H, Dk = v["rec_q"].shape
    Dv = v["rec_v"].shape[2]
    S = v["rec_S0"].copy()
    out["rec_o"] = ops.gdn_recurrent(S, v["rec_q"], v["rec_k"], v["rec_v"], v["rec_g"],
                                     v["rec_beta"], T, H, Dk, Dv)
    out["rec_S1"] = S
    out["on_y"] = ops.gdn_onorm(v["on_o"], v["on_z"], v["on_w"], 3, 32)
    out["rms_y"] = ops.attn_rmsnorm(v["rms_x"], v["rms_w"])
    out["rope_y"] = np.stack([ops.attn_rope(v["rope_x"], 64, float(p)) for p in v["rope_pos"]])
    Tq, H, D = v["gqa_q"].shape
    Tk, Hkv = v["gqa_k"].shape[:2]
    out["gqa_o"] = ops.attn_gqa(v["gqa_q"], v["gqa_k"], v["gqa_v"], Tq, Tk, H, Hkv, D,
                                float(1.0 / np.sqrt(D)))
    out["og_y"] = ops.attn_outgate(v["og_o"], v["og_gate"])
    return out


def _same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def test_oracle_ops_match_reference_vectors(orc, gv):
    out = _ops_outputs(orc, gv)
    bad = [k for k, a in out.items() if not _same_bits(a, gv[k].reshape(a.shape))]
    assert not bad, f"oracle differs from the reference vectors in {bad}"


def test_oracle_gdn_mixer_matches_reference_vectors(orc, gv):
    w = {k[5:]: gv[k] for k in gv if k.startswith("gm_w_")}
    conv, S = gv["gm_conv0"].copy(), gv["gm_S0"].copy()
    y = orc.gdn_mixer((2, 4, 16, 16), w, gv["gm_cu"], gv["gm_qkv"], gv["gm_z"], gv["gm_a"],
                      gv["gm_b"], conv, S)
    assert _same_bits(y, gv["gm_y"])
    assert _same_bits(conv, gv["gm_conv1"])
    assert _same_bits(S, gv["gm_S1"])


def test_oracle_attn_mixer_matches_reference_vectors(orc, gv):
    w = {k[5:]: gv[k] for k in gv if k.startswith("am_w_")}
    kc, vc = gv["am_kc0"].copy(), gv["am_vc0"].copy()
    y = orc.attn_mixer((4, 2, 64, 32, 1e7), w, gv["am_cu"], gv["am_pos0"], gv["am_qg"],
                       gv["am_k"], gv["am_v"], kc, vc, 16 * 2 * 64)
    assert _same_bits(y, gv["am_y"])
    assert _same_bits(kc, gv["am_kc1"]) and _same_bits(vc, gv["am_vc1"])


def test_golden_vectors_are_not_degenerate(gv):
    """The vectors exercise what they claim: nonzero outputs, the decay
    reaching its x>20 identity branch, state actually changed."""
    assert np.any(gv["conv_out"] != 0) and np.any(gv["gm_y"] != 0) and np.any(gv["am_y"] != 0)
    assert not np.array_equal(gv["rec_S0"], gv["rec_S1"])
    t = (gv["gate_a"].astype(np.uint32) << 16).view(np.float32) + gv["gate_dt"]
    assert np.any(t > 20.0) and np.any(t < 0.0)


@pytest.mark.gpu
def test_hip_ops_match_reference_vectors(hip, gv):
    out = _ops_outputs(hip, gv)
    for k, a in out.items():
        r = gv[k].reshape(np.asarray(a).shape)
        if a.dtype == np.uint16:
            assert_bf16_close(a, r, what=k)
        else:
            assert_state_close(a, r, what=k)


def test_oracle_gemm_matches_reference_vectors(orc, gv):
    for sfx in ("", "2"):
        y = orc.bf16_gemm(gv["gemm_w" + sfx], gv["gemm_x" + sfx])
        assert _same_bits(y, gv["gemm_y" + sfx])


@pytest.mark.gpu
def test_hip_gemm_matches_reference_vectors(hip, gv):
    """The projection drop-ins are bitwise the reference's (its order)."""
    for sfx in ("", "2"):
        w, x = gv["gemm_w" + sfx], gv["gemm_x" + sfx]
        assert _same_bits(hip.bf16_gemm(w, x), gv["gemm_y" + sfx])
        assert _same_bits(hip.bf16_gemv(w, np.ascontiguousarray(x[0])), gv["gemm_y" + sfx][0])
