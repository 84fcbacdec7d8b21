"""The C11 host (tests/c_host/host_layer.c, built by the csrc Makefile):
a C program includes include/apus_hip.h, binds libapus_hip.so through weak
references and drives one GDN and one GQA layer through tier 2 with the
reference's fail-soft hook pattern (c/bf16.h:199-205, 250-259).

CPU: built without the library the program links and takes the CPU path
("hip backend not linked"); linked, with APUS_HIP_DISABLE=1 it takes it
through the library's own refusal. GPU: every call runs on the device and
the results the C program wrote are checked against the oracle on the
inputs it wrote: GDN prefill (the chunked tolerance class) then decode
(the chunked prefill's state carried on: bf16 rows class, conv state bit-exact, state within 1e-4), GQA prefill then a verify step
(esc class, caches bit-exact).
"""
import os
import subprocess

import numpy as np
import pytest

import synth
from attn_util import attn_esc
from numerics import assert_bf16_esc, assert_bf16_rows, assert_state_close

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "tests", "c_host", "host_layer")
NOLIB = os.path.join(ROOT, "tests", "c_host", "host_layer_nolib")


def _run(exe, tmp_path, env=None):
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is not built: run __graft_entry__.build()")
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, **(env or {})))
    assert r.returncode == 0, r.stderr
    return r.stdout.strip()


def test_host_without_library_takes_cpu_path(tmp_path):
    assert _run(NOLIB, tmp_path) == "fallback init: hip backend not linked"


def test_host_disabled_takes_cpu_path(tmp_path):
    out = _run(HOST, tmp_path, {"APUS_HIP_DISABLE": "1"})
    assert out.startswith("fallback init:") and "APUS_HIP_DISABLE" in out


@pytest.mark.gpu
def test_host_layers_on_gpu(tmp_path, orc):
    out = _run(HOST, tmp_path)
    assert out == "hip", out

    def ld(name, dtype):
        return np.fromfile(tmp_path / f"{name}.bin", dtype=dtype)

    # GDN: prefill from zero state, then one decode token per sequence
    hk, hv, dk, dv = synth.GDN_DIMS
    cd, vd = 2 * hk * dk + hv * dv, hv * dv
    w = dict(conv_w=ld("gdn_conv_w", np.uint16).reshape(cd, 4), A_log=ld("gdn_A_log", np.float32),
             dt_bias=ld("gdn_dt_bias", np.float32), onorm_w=ld("gdn_onorm_w", np.uint16))
    cu_p = np.array([0, 70, 75, 108], np.int32)
    cu_d = np.array([0, 1, 2, 3], np.int32)
    conv = np.zeros((3, cd * 3), np.uint16)
    S = np.zeros((3, hv, dk, dv), np.float32)
    t = {n: ld(f"gdn_{n}_p", np.uint16) for n in ("qkv", "z", "a", "b")}
    y_p = orc.gdn_mixer(synth.GDN_DIMS, w, cu_p, t["qkv"].reshape(108, cd), t["z"].reshape(108, vd),
                        t["a"].reshape(108, hv), t["b"].reshape(108, hv), conv, S)
    t = {n: ld(f"gdn_{n}_d", np.uint16) for n in ("qkv", "z", "a", "b")}
    y_d = orc.gdn_mixer(synth.GDN_DIMS, w, cu_d, t["qkv"].reshape(3, cd), t["z"].reshape(3, vd),
                        t["a"].reshape(3, hv), t["b"].reshape(3, hv), conv, S)
    assert_bf16_rows(ld("gdn_y_p", np.uint16).reshape(108, vd), y_p, 128, what="C host gdn prefill")
    assert_bf16_rows(ld("gdn_y_d", np.uint16).reshape(3, vd), y_d, 128, what="C host gdn decode")
    assert np.array_equal(ld("gdn_conv", np.uint16).reshape(conv.shape), conv)
    assert_state_close(ld("gdn_S", np.float32).reshape(S.shape), S, what="C host gdn S")

    # GQA: prefill from position 0, then a verify step of 2 and 1 tokens
    nh, nkv, d, rot, theta = synth.ATTN_DIMS
    aw = dict(qn_w=ld("attn_qn_w", np.uint16), kn_w=ld("attn_kn_w", np.uint16))
    ms = 64
    kc = np.zeros((2, ms, nkv, d), np.uint16)
    vc = np.zeros((2, ms, nkv, d), np.uint16)
    steps = ((np.array([0, 40, 47], np.int32), np.array([0, 0], np.int32), "p", 47),
             (np.array([0, 2, 3], np.int32), np.array([40, 7], np.int32), "d", 3))
    for cu, pos0, tag, T in steps:
        tok = dict(qg=ld(f"attn_qg_{tag}", np.uint16).reshape(T, nh, 2 * d),
                   k=ld(f"attn_k_{tag}", np.uint16).reshape(T, nkv, d),
                   v=ld(f"attn_v_{tag}", np.uint16).reshape(T, nkv, d))
        y_o, qf, _ = orc.attn_mixer(synth.ATTN_DIMS, aw, cu, pos0, tok["qg"], tok["k"], tok["v"],
                                    kc, vc, ms * nkv * d, capture=True)
        esc = attn_esc(qf, kc, vc, cu, pos0, nh, nkv, d)
        assert_bf16_esc(ld(f"attn_y_{tag}", np.uint16).reshape(T, nh * d), y_o, esc, ulps=2,
                        what=f"C host attention {tag}")
    for s, n in ((0, 42), (1, 8)):
        assert np.array_equal(ld(f"attn_kc{s}", np.uint16).reshape(n, nkv, d), kc[s, :n])
        assert np.array_equal(ld(f"attn_vc{s}", np.uint16).reshape(n, nkv, d), vc[s, :n])
